"""Writes lamp3_known_answers.json beside this file: the literal inputs and
expected outputs of the reference's own tests for this path, transcribed by
hand (csrc/tests/tensor_tests.cpp, csrc/tests/autograd_tests.cpp,
tests/unit/test_module.py; each case names its file:line in "src").  Values
the gtests compute with std:: math (exp, log, cos, tan) are computed here in
float64 the same way.  Nothing here imports or runs the reference.

    python tests/golden/make_known_answers.py          # (re)write the fixture
    python tests/golden/make_known_answers.py --check  # exit 1 if it differs
"""
import json
import math
import sys
from pathlib import Path
A = [[1, 2], [3, 4], [5, 6]]
B = [[0.5, 1.5], [2.5, 3.5], [4.5, 5.5]]
a = [[1, 2], [3, 4], [5, 2]]
b = [[-1, 4], [-2, 0], [3, 0.5]]
inf = "inf"
def flat(x): return [v for r in x for v in r]
cases = {
 "tensor": [
  {"name": "scalar_broadcast", "src": "tensor_tests.cpp:100-113", "op": "add", "a": A, "b": [100.0], "shape": [3, 2], "expect": [101, 102, 103, 104, 105, 106]},
  {"name": "row_broadcast", "src": "tensor_tests.cpp:115-127", "op": "add", "a": A, "b": [[10, 20]], "shape": [3, 2], "expect": [11, 22, 13, 24, 15, 26]},
  {"name": "column_broadcast", "src": "tensor_tests.cpp:129-141", "op": "add", "a": A, "b": [[10], [20], [30]], "shape": [3, 2], "expect": [11, 12, 23, 24, 35, 36]},
  {"name": "reshape_broadcast", "src": "tensor_tests.cpp:143-170", "op": "add", "a": [[10, 20], [30, 40], [50, 60]], "b": [[10, 20]], "shape": [3, 2], "expect": [20, 40, 40, 60, 60, 80]},
  {"name": "expand_broadcast", "src": "tensor_tests.cpp:171-195", "op": "add", "a": [[[1], [2]], [[3], [4]], [[5], [6]]], "b": [[[7], [8]]], "shape": [3, 2, 1], "expect": [8, 10, 10, 12, 12, 14]},
  {"name": "expand_broadcast_reversed", "src": "tensor_tests.cpp:184-195", "op": "add", "a": [[[7], [8]]], "b": [[[1], [2]], [[3], [4]], [[5], [6]]], "shape": [3, 2, 1], "expect": [8, 10, 10, 12, 12, 14]},
  {"name": "pow_scalar", "src": "tensor_tests.cpp:554-579", "op": "pow", "a": A, "b": [2.0], "shape": [3, 2], "expect": [1, 4, 9, 16, 25, 36]},
  {"name": "pow_ones", "src": "tensor_tests.cpp:580-595", "op": "pow", "a": A, "b": [[1, 1], [1, 1], [1, 1]], "shape": [3, 2], "expect": flat(A)},
  {"name": "pow_zeros", "src": "tensor_tests.cpp:596-613", "op": "pow", "a": A, "b": [[0, 0], [0, 0], [0, 0]], "shape": [3, 2], "expect": [1] * 6},
  {"name": "eq", "src": "tensor_tests.cpp:616-627", "op": "eq", "a": A, "b": A, "shape": [3, 2], "expect": [1] * 6},
  {"name": "ne", "src": "tensor_tests.cpp:629-638", "op": "ne", "a": A, "b": B, "shape": [3, 2], "expect": [1] * 6},
  {"name": "lt", "src": "tensor_tests.cpp:640-649", "op": "lt", "a": A, "b": B, "shape": [3, 2], "expect": [0] * 6},
  {"name": "gt", "src": "tensor_tests.cpp:651-660", "op": "gt", "a": A, "b": B, "shape": [3, 2], "expect": [1] * 6},
  {"name": "le", "src": "tensor_tests.cpp:662-674", "op": "le", "a": A, "b": A, "shape": [3, 2], "expect": [1] * 6},
  {"name": "ge", "src": "tensor_tests.cpp:676-687", "op": "ge", "a": A, "b": A, "shape": [3, 2], "expect": [1] * 6},
  {"name": "broadcast_pow_row", "src": "tensor_tests.cpp:706-720", "op": "pow", "a": A, "b": [[1, 2]], "shape": [3, 2], "expect": [1, 4, 3, 16, 5, 36], "atol": 1e-4},
  {"name": "broadcast_gt_row", "src": "tensor_tests.cpp:723-732", "op": "gt", "a": A, "b": [[10, 20]], "shape": [3, 2], "expect": [0] * 6},
  {"name": "broadcast_ge_scalar", "src": "tensor_tests.cpp:734-741", "op": "ge", "a": A, "b": [3.5], "shape": [3, 2], "expect": [0, 0, 0, 1, 1, 1]},
  {"name": "broadcast_lt_col", "src": "tensor_tests.cpp:743-752", "op": "lt", "a": A, "b": [[10], [20], [30]], "shape": [3, 2], "expect": [1] * 6},
 ],
 "reduce": [
  {"name": "sum_axis0", "src": "tensor_tests.cpp:196-212", "op": "sum", "a": A, "axis": 0, "shape": [1, 2], "expect": [9, 12]},
  {"name": "sum_axis1", "src": "tensor_tests.cpp:213-224", "op": "sum", "a": A, "axis": 1, "shape": [3, 1], "expect": [3, 7, 11]},
 ],
 "autograd": [
  {"name": "add", "src": "autograd_tests.cpp:51-66", "expr": "a + b", "out": [0, 6, 1, 4, 8, 2.5], "grad_a": [1] * 6, "grad_b": [1] * 6},
  {"name": "sub", "src": "autograd_tests.cpp:68-82", "expr": "a - b", "out": [2, -2, 5, 4, 2, 1.5], "grad_a": [1] * 6, "grad_b": [-1] * 6},
  {"name": "mul", "src": "autograd_tests.cpp:84-98", "expr": "a * b", "out": [-1, 8, -6, 0, 15, 1], "grad_a": flat(b), "grad_b": flat(a)},
  {"name": "div", "src": "autograd_tests.cpp:100-122", "expr": "a / b", "out": [-1, 0.5, -1.5, inf, 5 / 3, 4],
   "grad_a": [1 / -1, 1 / 4, 1 / -2, inf, 1 / 3, 1 / 0.5],
   "grad_b": [-1 / 1, -2 / 16, -3 / 4, "-inf", -5 / 9, -2 / 0.25]},
  {"name": "exp", "src": "autograd_tests.cpp:124-134", "expr": "exp(b)", "out": [math.exp(v) for v in flat(b)], "grad_b": [math.exp(v) for v in flat(b)]},
  {"name": "log", "src": "autograd_tests.cpp:136-146", "expr": "log(a)", "out": [math.log(v) for v in flat(a)], "grad_a": [1 / v for v in flat(a)]},
  {"name": "matmul", "src": "autograd_tests.cpp:229-248", "expr": "a @ m", "m": [[-1], [4]], "out": [7, 13, 3], "grad_a": [-1, 4, -1, 4, -1, 4], "grad_m": [9, 8]},
  {"name": "transpose", "src": "autograd_tests.cpp:250-263", "expr": "transpose(a)", "out": [1, 3, 5, 2, 4, 2], "grad_a": [1] * 6},
  {"name": "sum1", "src": "autograd_tests.cpp:265-277", "expr": "sum(a, 1)", "out": [3, 7, 7], "grad_a": [1] * 6},
  {"name": "max1", "src": "autograd_tests.cpp:279-291", "expr": "max(a, 1)", "out": [2, 4, 5], "grad_a": [0, 1, 0, 1, 1, 0]},
  {"name": "min1", "src": "autograd_tests.cpp:293-305", "expr": "min(a, 1)", "out": [1, 3, 2], "grad_a": [1, 0, 1, 0, 0, 1]},
  {"name": "broadcast_add", "src": "autograd_tests.cpp:360-385", "expr": "a + r", "r": [[10, 20]], "out": [11, 22, 13, 24, 15, 22], "grad_a": [1] * 6, "grad_r": [3, 3]},
 ],
 "autograd_unary": [
  {"name": "sqrt", "src": "autograd_tests.cpp:148-158", "fn": "sqrt", "x": [0.25, 1, 4, 9], "grad": [1, 0.5, 0.25, 1 / 6]},
  {"name": "cos", "src": "autograd_tests.cpp:160-171", "fn": "cos", "x": [-1, 0, 0.5, 1], "grad": [-math.sin(v) for v in [-1, 0, 0.5, 1]]},
  {"name": "tan", "src": "autograd_tests.cpp:173-186", "fn": "tan", "x": [-0.75, -0.25, 0, 0.5], "grad": [1 + math.tan(v) ** 2 for v in [-0.75, -0.25, 0, 0.5]]},
  {"name": "clamp_strict", "src": "autograd_tests.cpp:205-215", "fn": "clamp", "lo": -1, "hi": 1, "x": [-2, -1, 0, 1, 2], "grad": [0, 0, 1, 0, 0]},
  {"name": "abs", "src": "autograd_tests.cpp:217-227", "fn": "abs", "x": [-2, 0, 3], "grad": [-1, 0, 1]},
 ],
 "inputs": {"a": a, "b": b, "src": "autograd_tests.cpp:31-40"},
 "repeated_backward": {"src": "autograd_tests.cpp:487-499", "expr": "a * 2.0, backward twice", "grad_a": [4] * 6},
 "functional_sgd": {"src": "tests/unit/test_module.py:161-192", "w": [1.0, 2.0], "x": [1.0, 1.0], "y": [3.0, 5.0], "lr": 0.1, "expect": [1.4, 2.6]},
 "tolerance": {"atol": 1e-5, "src": "tensor_tests.cpp:19, autograd_tests.cpp:20"},
}
OUT = Path(__file__).resolve().parent / "lamp3_known_answers.json"

if __name__ == "__main__":
    text = json.dumps(cases, indent=1)
    if "--check" in sys.argv[1:]:
        sys.exit(0 if json.loads(OUT.read_text()) == json.loads(text) else 1)
    OUT.write_text(text)
