from .activation import ReLU, Sigmoid, Softmax, Tanh
from .container import Sequential
from .dropout import Dropout
from .linear import Flatten, Linear

__all__ = ["ReLU", "Sigmoid", "Softmax", "Tanh", "Sequential", "Dropout",
           "Flatten", "Linear"]
