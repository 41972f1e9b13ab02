"""bench.py's contract and its profile summarizers, on the CPU: --gpus N > 1
is refused with a message, and the rocprofv3 summaries are recomputed from the
synthetic CSV fixtures of tests/golden/rocprof (made by make_fixtures.py)."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
FIX = ROOT / "tests" / "golden" / "rocprof"


def run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_traffic_summary_scales_counters_by_the_copy_calibration(tmp_path):
    r = run("--summarize", str(FIX / "stats"), str(FIX / "fetch"), str(FIX / "write"), str(FIX / "copy_fetch"),
            str(FIX / "copy_write"), "fixture", "--profiles-dir", str(tmp_path))
    assert r.returncode == 0, r.stderr
    out = json.loads((tmp_path / "fixture_traffic.json").read_text())
    # FETCH scale = 512 MiB / 262144 KiB = 2; WRITE scale 1.
    assert out["fetch_scale"] == 2.0 and out["write_scale"] == 1.0
    # (150000 * 2 + 1000 * 2) KiB read + (2000 + 200) KiB written, per op call
    assert out["hbm_bytes_per_launch"] == (302000 + 2200) * 1024
    assert abs(out["op_time_us_rocprof"] - 55.5) < 1e-9
    md = (tmp_path / "fixture.md").read_text()
    assert "decodeKernel<false, 2>" in md and "rocprofv3 --pmc FETCH_SIZE" in md


def test_step_summary_takes_the_last_steps(tmp_path):
    r = run("--summarize-step", str(FIX / "trace"), "steps", "--steps", "2", "--profiles-dir", str(tmp_path))
    assert r.returncode == 0, r.stderr
    md = (tmp_path / "steps.md").read_text()
    # each step: 4 + 9 + 4 us of kernels with 0.5 us after each; the span of
    # the last two steps runs from the first kernel's start to the last's end
    import re

    assert "kernels busy 17.0 us per step" in md
    span = float(re.search(r"GPU span ([0-9.]+) us per step", md).group(1))
    assert abs(span - (18.5 + 18.0) / 2) < 0.06
    assert "hipBLASLt GEMM MT32x32x128" in md
