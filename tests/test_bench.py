"""bench.py's host-side contract (no GPU): more than one GPU is refused with a message, and the roofline traffic
figure comes from the committed rocprofv3 counter summary, scaled by the copy calibration it records."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_traffic_from_committed_counters():
    sys.path.insert(0, str(ROOT))
    import bench

    t = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    cal = t["copy_calibration"]
    k = t["kernels"]["attn_fwd_dma_kernel<BF16, 128"]
    want = int(k["FETCH_SIZE_KiB"] / cal["FETCH_SIZE_KiB"] * cal["bytes_read"]
               + k["WRITE_SIZE_KiB"] / cal["WRITE_SIZE_KiB"] * cal["bytes_written"])
    got = bench.measured_traffic("attn_fwd_dma_kernel<BF16, 128")
    assert got == want
    # config 2 moves at least its algorithmic bytes (q, k, v read once, o written once: 134.2 MB) and, with the
    # K/V prefix re-reads of the 16 query tiles mostly served by L2, well under twice that
    assert 134_217_728 <= got < 2 * 134_217_728
    assert bench.measured_traffic("no_such_kernel") is None
