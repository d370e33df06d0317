"""Build recipe for the native parts, in-tree.

Outputs
  ormi_amd/lib/libormi_hip.so      HIP device layer (hipcc, gfx950), C ABI of include/ormi_hip.h
  ormi_amd/lib/libormi_core.so     graph, autograd, runtime, HIP backend host code (g++)
  ormi_amd/ormi_backend*.so        pybind11 module (g++)
  oracle/_build/libormi_cpu_oracle.so  CPU oracle, test infrastructure only (g++)
  oracle/_ref/libormi_ref.so       the reference's own CPU path, a second checker, and
  oracle/_ref/libormi_ref_hip.so   the reference's core with the HIP device plugged in over
                                   libormi_hip.so (make -f oracle/Makefile.ref; built where
                                   /root/reference exists, and shipped prebuilt elsewhere)

Run `python -m ormi_amd._build` (or __graft_entry__.build()). Every call
recompiles everything; objects go to ormi_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIBDIR = PKG / "lib"
OBJDIR = PKG / "_build"
GENDIR = OBJDIR / "gen"
ORACLE = ROOT / "oracle"
REF_CSRC = Path("/root/reference/ormi-core/csrc")  # reference sources: read and compiled, never copied
ORACLE_OUT = ORACLE / "_build"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = os.environ.get("ORMI_HIP_ARCH", "gfx950")

# Every HIP translation unit: gfx950 only, packed-FP32 instructions disabled,
# no FP contraction (the generated kernels' setting, so GEMM epilogues round
# like the element-wise kernels they replace).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f'-DORMI_HIP_TARGET="{ARCH}"',  # ormi_hip_init refuses a device of another architecture
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function"]

CORE_SOURCES = sorted(
    [p for p in (CSRC / "core").rglob("*.cpp")]
    + [p for p in (CSRC / "runtime").rglob("*.cpp")]
    + [p for p in (CSRC / "backend").rglob("*.cpp")]
)
HIP_SOURCES = sorted((CSRC / "hip").glob("*.hip"))
# Host C++ of the device layer: the C-ABI reduction and map entries and the code
# generator they share with the core (a second, hidden-symbol copy inside
# libormi_hip.so).
DEVICE_HOST_SOURCES = [CSRC / "hip" / "reduce_entry.cpp", CSRC / "hip" / "map_entry.cpp",
                       CSRC / "backend" / "hip" / "codegen.cpp",
                       CSRC / "core" / "dtype.cpp", CSRC / "core" / "ops.cpp"]
BINDING_SOURCES = sorted((CSRC / "bindings").glob("*.cpp"))
ORACLE_SOURCES = sorted((ORACLE / "cpu_backend").glob("*.cpp"))

EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
MODULE_PATH = PKG / f"ormi_backend{EXT_SUFFIX}"
HIP_LIB = LIBDIR / "libormi_hip.so"
CORE_LIB = LIBDIR / "libormi_core.so"
ORACLE_LIB = ORACLE_OUT / "libormi_cpu_oracle.so"


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, cwd=cwd)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip() and os.environ.get("ORMI_BUILD_VERBOSE"):
        print(out)


def _gen_device_text() -> None:
    """Embed the device helper header as a raw string for the hipRTC generator."""
    GENDIR.mkdir(parents=True, exist_ok=True)
    text = (CSRC / "hip" / "device" / "ormi_device.h").read_text()
    delim = "ORMIDEV"
    assert f"){delim}\"" not in text
    (GENDIR / "ormi_device_text.inc").write_text(f'R"{delim}({text}){delim}"\n')


_INCREMENTAL = False


def _newest_header() -> float:
    heads = [p for d in (CSRC, INCLUDE) for p in d.rglob("*.h")]
    return max((p.stat().st_mtime for p in heads), default=0.0)


def _fresh(src: Path, obj: Path) -> bool:
    """Incremental builds only: obj is newer than its source and every header."""
    if not _INCREMENTAL or not obj.exists():
        return False
    t = obj.stat().st_mtime
    return t > src.stat().st_mtime and t > _newest_header()


def _compile_cxx(src: Path, includes: list[Path], extra: list[str] | None = None, tag: str = "") -> Path:
    rel = src.relative_to(ROOT)
    obj = OBJDIR / "obj" / (str(rel).replace(os.sep, "__") + tag + ".o")
    obj.parent.mkdir(parents=True, exist_ok=True)
    if _fresh(src, obj):
        return obj
    cmd = ["g++", *CXX_FLAGS, *(extra or []), *[f"-I{p}" for p in includes], "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def _compile_hip(src: Path) -> Path:
    obj = OBJDIR / "obj" / (str(src.relative_to(ROOT)).replace(os.sep, "__") + ".o")
    obj.parent.mkdir(parents=True, exist_ok=True)
    if _fresh(src, obj):
        return obj
    _run([HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC / 'hip'}", "-c", str(src), "-o", str(obj)])
    return obj


def build(verbose: bool = False, incremental: bool = False) -> None:
    """Compile every part. incremental=True (python -m ormi_amd._build -i) skips
    objects newer than their source and every header; the default recompiles all."""
    global _INCREMENTAL
    _INCREMENTAL = incremental
    if verbose:
        os.environ["ORMI_BUILD_VERBOSE"] = "1"
    LIBDIR.mkdir(parents=True, exist_ok=True)
    ORACLE_OUT.mkdir(parents=True, exist_ok=True)
    _gen_device_text()

    core_inc = [CSRC, INCLUDE, GENDIR]
    import pybind11

    py_inc = [Path(sysconfig.get_paths()["include"]), Path(pybind11.get_include())]
    jobs = int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))
    jobs = max(1, min(jobs, 16))

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        # One object per HIP translation unit, compiled in parallel (the GEMM
        # units take the longest), then linked into the shared library.
        hip_objs = [ex.submit(_compile_hip, s) for s in HIP_SOURCES]
        dev_host_objs = [ex.submit(_compile_cxx, s, core_inc + [CSRC / "hip"], ["-fvisibility=hidden"], ".dev")
                         for s in DEVICE_HOST_SOURCES]
        core_objs = [ex.submit(_compile_cxx, s, core_inc) for s in CORE_SOURCES]
        bind_objs = [ex.submit(_compile_cxx, s, core_inc + py_inc) for s in BINDING_SOURCES]
        oracle_objs = [ex.submit(_compile_cxx, s, core_inc) for s in ORACLE_SOURCES]
        hip = [f.result() for f in hip_objs] + [f.result() for f in dev_host_objs]
        core = [f.result() for f in core_objs]
        binds = [f.result() for f in bind_objs]
        oracle = [f.result() for f in oracle_objs]

    _run([HIPCC, *HIP_FLAGS, "-shared", *map(str, hip), "-o", str(HIP_LIB), "-lhiprtc", f"-Wl,-rpath,{ROCM / 'lib'}"])
    _run(["g++", "-shared", *map(str, core), "-o", str(CORE_LIB), "-Wl,-soname,libormi_core.so", f"-L{LIBDIR}", "-lormi_hip",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,--no-undefined"])
    _run(["g++", "-shared", *map(str, binds), "-o", str(MODULE_PATH), f"-L{LIBDIR}", "-lormi_core", "-lormi_hip",
          "-Wl,-rpath,$ORIGIN/lib"])
    rel_lib = os.path.relpath(LIBDIR, ORACLE_OUT)
    _run(["g++", "-shared", *map(str, oracle), "-o", str(ORACLE_LIB), f"-L{LIBDIR}", "-lormi_core",
          f"-Wl,-rpath,$ORIGIN/{rel_lib}", "-Wl,--no-undefined"])
    # The reference's own CPU path, a second checker for the oracle, where its
    # sources are (this container; other machines use the prebuilt file).
    if REF_CSRC.is_dir():
        _run(["make", "-s", "-j2", "-f", "oracle/Makefile.ref", f"REF={REF_CSRC}"] + ([] if incremental else ["-B"]), cwd=ROOT)


def built() -> bool:
    return HIP_LIB.exists() and CORE_LIB.exists() and MODULE_PATH.exists()


if __name__ == "__main__":
    build(verbose="-v" in sys.argv, incremental="-i" in sys.argv)
    print("built:", HIP_LIB, CORE_LIB, MODULE_PATH, ORACLE_LIB)
