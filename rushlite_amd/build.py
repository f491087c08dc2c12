"""Build recipe for the MI355X backend, the Python extension and the oracle.

Outputs (all in-tree so they travel with the repository snapshot):
  rushlite_amd/lib/liblmp_hip.so      C-ABI HIP backend (hipcc, gfx950)
  rushlite_amd/_C.<abi>.so             Lamp3 host framework + pybind11 module
  oracle/liblamp_cpu.so               CPU oracle, strict IEEE (test only)
  oracle/liblamp_cpu_fast.so          CPU oracle with the reference's flags (AVX2 + FMA)
  oracle/liblamp_cpu_fast_v4.so       the same for AVX-512 hosts

Run ``python rushlite_amd/build.py [all|hip|ext|oracle]`` from the repository
root (or ``__graft_entry__.build()``).  It imports nothing from the package, so
it also runs in a fresh checkout, where importing ``rushlite_amd`` (and with it
``python -m rushlite_amd.build``) fails until the extension exists.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
HIP_SRC = PKG / "csrc" / "hip"
CORE_SRC = PKG / "csrc" / "core"
BIND_SRC = PKG / "csrc" / "bindings"
BUILD = ROOT / "_build"
LIB = PKG / "lib"
ORACLE = ROOT / "oracle"

ARCH = os.environ.get("LMP_HIP_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
CC = os.environ.get("CC", "gcc")

# -ffp-contract=off: eager Lamp3 rounds after every op; no FMA contraction.
# packed-fp32-ops disabled: the compiler must not form v_pk_* fp32 ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-parameter",
             "-fvisibility=hidden"]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and "unknown target feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}):\n"
                           f"{' '.join(cmd)}\n{out}")


def _parallel(jobs: list[list[str]], workers: int | None = None) -> None:
    workers = workers or min(8, os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for f in [ex.submit(_run, j) for j in jobs]:
            f.result()


def build_hip() -> Path:
    """Compile csrc/hip/*.hip into rushlite_amd/lib/liblmp_hip.so."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    obj_dir = BUILD / "hip"
    obj_dir.mkdir(parents=True, exist_ok=True)
    LIB.mkdir(parents=True, exist_ok=True)
    srcs = sorted(HIP_SRC.glob("*.hip"))
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    _parallel([[HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)]
               for s, o in zip(srcs, objs)])
    out = LIB / "liblmp_hip.so"
    tmp = LIB / "liblmp_hip.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), "-lhiprtc", "-Wl,-soname,liblmp_hip.so"])
    os.replace(tmp, out)
    return out


def build_ext() -> Path:
    """Compile the host framework + bindings into the _C extension module."""
    import pybind11

    obj_dir = BUILD / "core"
    obj_dir.mkdir(parents=True, exist_ok=True)
    py_inc = sysconfig.get_paths()["include"]
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    incs = [f"-I{INCLUDE}", f"-I{CORE_SRC}", f"-I{py_inc}",
            f"-I{pybind11.get_include()}"]
    srcs = sorted(CORE_SRC.glob("*.cpp")) + sorted(BIND_SRC.glob("*.cpp"))
    objs = [obj_dir / (s.parent.name + "_" + s.stem + ".o") for s in srcs]
    _parallel([[CXX, *CXX_FLAGS, *incs, "-c", str(s), "-o", str(o)]
               for s, o in zip(srcs, objs)])
    out = PKG / f"_C{suffix}"
    tmp = PKG / f"_C{suffix}.tmp"
    _run([CXX, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          f"-L{LIB}", "-llmp_hip", "-Wl,-rpath,$ORIGIN/lib",
          "-Wl,--no-as-needed"])
    os.replace(tmp, out)
    return out


def build_oracle() -> list[Path]:
    """Compile the CPU oracle: strict IEEE (parity) and the reference's
    -O3 -ffast-math flags (timed baseline), the latter for two ISA levels."""
    src = ORACLE / "lamp_cpu.c"
    # Named ISA levels rather than -march=native: the libraries are built here
    # and loaded on the GPU host, whose CPU differs.  The loader takes the
    # x86-64-v4 (AVX-512) fast build where the host's CPU flags allow it, which
    # is what -march=native gives on such a host, and x86-64-v3 (AVX2 + FMA)
    # otherwise.  -mno-daz-ftz keeps gcc from linking its fast-math startup
    # code into the fast builds: it would set flush-to-zero in every process
    # that loads them (numpy included); the baseline sets that mode for its
    # timed region itself (lcpu_set_denormal_flush).
    common = [CC, "-O3", "-fopenmp", "-fPIC", "-shared", "-std=c11"]
    jobs = [
        [*common, "-march=x86-64-v3", "-ffp-contract=off", str(src), "-o",
         str(ORACLE / "liblamp_cpu.so"), "-lm"],
        [*common, "-march=x86-64-v3", "-ffast-math", "-mno-daz-ftz", str(src), "-o",
         str(ORACLE / "liblamp_cpu_fast.so"), "-lm"],
        [*common, "-march=x86-64-v4", "-ffast-math", "-mno-daz-ftz", str(src), "-o",
         str(ORACLE / "liblamp_cpu_fast_v4.so"), "-lm"],
    ]
    _parallel(jobs)
    return [ORACLE / "liblamp_cpu.so", ORACLE / "liblamp_cpu_fast.so",
            ORACLE / "liblamp_cpu_fast_v4.so"]


def build_all() -> None:
    build_oracle()
    build_hip()
    build_ext()


if __name__ == "__main__":
    what = sys.argv[1:] or ["all"]
    for w in what:
        {"all": build_all, "hip": build_hip, "ext": build_ext,
         "oracle": build_oracle}[w]()
    print("built:", ", ".join(what))
