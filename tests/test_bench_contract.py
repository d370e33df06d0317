"""bench.py's JSON fields that come from committed files, checked without a GPU."""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_roofline_traffic_comes_from_the_committed_counter_summary():
    """roofline.traffic is the C2 kernel's read + write bytes per launch from
    profiles/hbm_traffic.md (the --pmc-report row the bench names); it must be
    found, and lie within 1% of the algorithmic bytes."""
    t = bench.traffic_from_profile("C2 fused map")
    assert isinstance(t, int)
    assert abs(t - bench.c2_bytes()) <= 0.01 * bench.c2_bytes()


def test_gpus_above_one_exit_with_a_message(capsys, monkeypatch):
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "2"])
    try:
        bench.main()
    except SystemExit as e:
        assert e.code == 2
    else:
        raise AssertionError("bench.py --gpus 2 did not exit")
    assert "one GPU" in capsys.readouterr().err
