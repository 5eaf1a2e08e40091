"""bench.py's driver contract, checked on the CPU (no GPU, no torch import).

- ``--gpus N`` with N > 1 exits non-zero with a JSON line saying that this
  build measures one GPU;
- the roofline ``traffic`` figure bench.py reports is read from the committed
  rocprofv3 summary of the headline kernel, and it is close to (not below)
  the kernel's algorithmic bytes per launch.
"""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_headline_traffic_is_read_from_profile():
    import bench
    t = bench.measured_traffic()
    assert isinstance(t, int)
    # Hkv 16 x L 32768 x 2 (K and V) x (128 B nibbles + 4 x 4 B fp16 scale/bias)
    # + q (32 x 256 bf16) + out (32 x 256 f32): the headline's algorithmic bytes.
    algorithmic = 16 * 32768 * 2 * (128 + 16) + 32 * 256 * 2 + 32 * 256 * 4
    assert algorithmic == 151_044_096
    assert algorithmic <= t <= 1.1 * algorithmic
