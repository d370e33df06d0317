"""bench.py's register-only MFMA probe (the matrix-core ceilings behind the
GEMM rooflines) and its HBM stream probe (the read, copy and write ceilings
behind the element-wise and reduction rooflines) compile for gfx950 through
libormi_hip's hipRTC, so the ceiling tables can be regenerated from the
repository (no GPU needed here)."""
import ctypes
import importlib.util
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_mfma_probe_source_compiles(cabi):
    spec = importlib.util.spec_from_file_location("ormi_bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    size = ctypes.c_size_t(0)
    rc = cabi.ormi_hip_rtc_compile_only(bench.MFMA_PROBE_SRC.encode(), b"gfx950", None, 0, ctypes.byref(size))
    assert rc == 0, cabi.ormi_hip_last_error()
    assert size.value > 0
    v = bench.mfma_probe_values()
    assert v.shape == (4096,) and len(set(v[:512].tolist())) > 400


def test_hbm_probe_source_compiles(cabi):
    spec = importlib.util.spec_from_file_location("ormi_bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    size = ctypes.c_size_t(0)
    rc = cabi.ormi_hip_rtc_compile_only(bench.HBM_PROBE_SRC.encode(), b"gfx950", None, 0, ctypes.byref(size))
    assert rc == 0, cabi.ormi_hip_last_error()
    assert size.value > 0
