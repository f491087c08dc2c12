"""CPU-only checks of the boundary and of host-side native logic.

* liblmp_hip.so loads without a GPU and exports every entry point declared in
  include/lmp_hip.h (and the ctypes mirror covers all of them);
* the caching arena and the magic-number divider, compiled from the backend's
  own headers with g++ and exercised against exact answers;
* the Python package imports and fails loudly (RuntimeError naming the
  missing device) when a GPU op runs without a GPU.
"""
import ctypes
import re
import shutil
import sys
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "lmp_hip.h"
HIP_SRC = ROOT / "rushlite_amd" / "csrc" / "hip"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lmp_(?:rt|k|jit)_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert len(names) == 44
    for group in ("lmp_rt_malloc", "lmp_rt_kernel_launch_count", "lmp_k_binary", "lmp_k_reduce",
                  "lmp_k_gemm_f32",
                  "lmp_jit_compile", "lmp_rt_graph_begin", "lmp_rt_graph_launch",
                  "lmp_k_gemm_f32_noalloc", "lmp_k_gemm_colsum_masked_f32",
                  "lmp_k_linear_backward_f32"):
        assert group in names


def test_library_exports_every_declared_symbol():
    from rushlite_amd import abi
    lib = ctypes.CDLL(str(abi.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(abi.SIGNATURES)
    abi.lib()  # argtypes/restype binding succeeds for every entry
    assert abi.lib().lmp_rt_abi_version() == 9


def test_build_recipe_imports_nothing_from_the_package():
    """rushlite_amd/build.py must run in a fresh checkout, where importing the
    package fails until the extension it builds exists: it imports nothing
    from the package, and __graft_entry__.build() loads it by path."""
    import ast
    tree = ast.parse((ROOT / "rushlite_amd" / "build.py").read_text())
    mods = set()
    for node in ast.walk(tree):
        if isinstance(node, ast.Import):
            mods.update(a.name.split(".")[0] for a in node.names)
        elif isinstance(node, ast.ImportFrom):
            assert node.level == 0, "relative import in build.py"
            mods.add((node.module or "").split(".")[0])
    assert "rushlite_amd" not in mods and "oracle" not in mods
    # beyond the standard library only the binding generator's include paths
    assert mods - set(sys.stdlib_module_names) <= {"pybind11"}
    entry = (ROOT / "__graft_entry__.py").read_text()
    assert "spec_from_file_location" in entry and "from rushlite_amd import build" not in entry


def test_gemm_entries_refuse_extents_near_2_31():
    """Every GEMM entry point refuses an extent or leading dimension of
    2^31 - 4096 or more (LMP_ERR_UNSUPPORTED) while validating its arguments,
    before it touches the device: the kernels' tile, fragment and K-loop
    indices are ints that reach a few thousand past an extent.  The operand
    pointers are placeholders that nothing reads, so the test runs only where
    no GPU is visible."""
    from conftest import gpu_available
    if gpu_available():
        pytest.skip("placeholder pointers: argument validation is checked on a host without a GPU")
    from rushlite_amd import abi
    L = abi.lib()
    big, p = (1 << 31) - 4096, 4096  # p: a non-null placeholder address
    for ta in (0, 1):
        for tb in (0, 1):
            for m, n, k in ((big, 8, 8), (8, big, 8), (8, 8, big)):
                lda = (m if ta else k)
                ldb = (k if tb else n)
                assert L.lmp_k_gemm_f32(ta, tb, m, n, k, p, lda, p, ldb, p, n, 0) == abi.ERR_UNSUPPORTED
                assert L.lmp_k_gemm(abi.FLOAT64, ta, tb, m, n, k,
                                    p, lda, p, ldb, p, n, 0) == abi.ERR_UNSUPPORTED
    # a leading dimension alone at the limit
    assert L.lmp_k_gemm_f32(0, 0, 8, 8, 8, p, big, p, 8, p, 8, 0) == abi.ERR_UNSUPPORTED
    assert L.lmp_k_linear_f32(0, 0, 8, big, 8, p, 8, p, big, p, p, big) == abi.ERR_UNSUPPORTED
    assert L.lmp_k_linear_relu_f32(0, 0, 8, big, 8, p, 8, p, big, p, p, big) == abi.ERR_UNSUPPORTED
    assert L.lmp_k_gemm_colsum_f32(1, 0, 8, 8, big, p, 8, p, 8, p, 8, 0, p, 0) == abi.ERR_UNSUPPORTED
    assert L.lmp_k_gemm_colsum_masked_f32(1, 8, 8, big, p, 8, p, p, 8, p, 8, 0, p, 0) == abi.ERR_UNSUPPORTED
    assert L.lmp_k_linear_backward_f32(big, 8, 8, p, 8, p, 8, p, 8, p, 8, 0, p, 8, 0, p, 0) == abi.ERR_UNSUPPORTED


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
@pytest.mark.parametrize("sanitize", [None, "thread"], ids=["plain", "tsan"])
def test_arena_fastdiv_and_copy_pool(tmp_path, sanitize):
    """The arena, its growth policy, the divider and the staged copies' host
    thread pool; once more under ThreadSanitizer for the pool's hand-offs."""
    exe = tmp_path / "host_check"
    flags = ["-O1", "-g", f"-fsanitize={sanitize}"] if sanitize else ["-O2"]
    build = subprocess.run(["g++", *flags, "-std=c++20", "-pthread", f"-I{HIP_SRC}",
                            str(ROOT / "tests" / "native" / "host_check.cpp"), "-o", str(exe)],
                           capture_output=True, text=True)
    if sanitize and build.returncode != 0:
        pytest.skip(f"g++ cannot build with -fsanitize={sanitize} here")
    assert build.returncode == 0, build.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "host checks ok" in out.stdout
    assert "WARNING: ThreadSanitizer" not in out.stderr, out.stderr


def test_package_imports_and_gpu_ops_fail_loudly_without_gpu():
    import rushlite_amd as rsl
    assert rsl.device.cuda == rsl.device.hip
    assert {"capture_on", "capture", "no_grad", "Module", "Variable"} <= set(rsl.__all__)
    from rushlite_amd.nets import layers  # noqa: F401
    if rsl.hip.is_available():
        pytest.skip("a GPU is present; the no-GPU failure path does not apply")
    with pytest.raises(RuntimeError, match="HIP device"):
        rsl.Variable([1.0, 2.0])


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fusion_codegen_compiles_with_hiprtc(tmp_path):
    """The kernels the fusion backend generates (elementwise and row regions)
    compile with hipRTC for gfx950; runs on the host without a GPU, over
    storage-less device leaves, linked with the framework objects the
    extension build leaves in _build/core."""
    objs = sorted((ROOT / "_build" / "core").glob("core_*.o"))
    hiprtc = Path("/opt/rocm/lib/libhiprtc.so")
    if not objs or not hiprtc.exists():
        pytest.skip("needs the built framework objects and ROCm's hipRTC")
    exe = tmp_path / "fusion_codegen"
    lib = ROOT / "rushlite_amd" / "lib"
    subprocess.run(["g++", "-O1", "-std=c++20", f"-I{ROOT / 'include'}",
                    f"-I{ROOT / 'rushlite_amd' / 'csrc' / 'core'}", "-I/opt/rocm/include",
                    "-D__HIP_PLATFORM_AMD__", str(ROOT / "tests" / "native" / "fusion_codegen.cpp"),
                    *map(str, objs), f"-L{lib}", "-llmp_hip", "-L/opt/rocm/lib", "-lhiprtc",
                    f"-Wl,-rpath,{lib}:/opt/rocm/lib", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout[-3000:] + out.stderr[-2000:]
    assert "fusion codegen ok" in out.stdout


def test_sequence_constructor_shapes_and_errors():
    """Variable(nested sequence) on the CPU device: the shape numpy derives,
    numbers of any kind as their float64 values, one number as a [1] tensor,
    and Lamp3's two error texts for ragged nesting and non-numeric items
    (bindings/variable.hpp:21-48)."""
    import rushlite_amd as rsl
    cpu = rsl.device.cpu
    for data, shape, values in (([[1, 2], [3, 4]], [2, 2], [1.0, 2.0, 3.0, 4.0]),
                                (((1, 2), (3, 4)), [2, 2], [1.0, 2.0, 3.0, 4.0]),
                                ([1.5, True, 3], [3], [1.5, 1.0, 3.0]),
                                (2.5, [1], [2.5]), ([], [0], []), ([[]], [1, 0], []),
                                ([2**70, 1], [2], [float(2**70), 1.0]),
                                ([[2**64], [-(2**65)]], [2, 1], [float(2**64), -float(2**65)])):
        v = rsl.Variable(data, device=cpu)
        assert v.shape == shape and v.data.tolist() == values, data
    for bad in ([[1, 2], [3]], [[1, 2], 3]):
        with pytest.raises(ValueError, match="Rushlite: array must be uniform"):
            rsl.Variable(bad, device=cpu)
    for bad in ([1, "a"], [1, None], "abc", [1 + 2j], [2**70, None], [2**70, "a"],
                [2**70, 1 + 2j]):
        with pytest.raises(ValueError, match="Rushlite: invalid input type"):
            rsl.Variable(bad, device=cpu)
