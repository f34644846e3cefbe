"""bench.py's contract pieces that need no GPU: the one-GPU guard, the algorithmic bytes per
expert, and the committed rocprofv3 traffic summary it reads."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_bytes_per_expert_at_gptoss_shapes():
    # gate_up codes 8,294,400 + scales 518,400 + down codes 4,147,200 + scales 259,200 +
    # biases (2I + H) x 2 = 17,280
    assert bench.bytes_per_expert(2880, 2880, True) == 13_236_480
    assert bench.bytes_per_expert(2880, 2880, False) == 13_219_200
    assert bench.gate_up_bytes_per_expert(2880, 2880, True) == 8_294_400 + 518_400 + 11_520
    # fine-grained layer (H=7168, I=2048, no biases): 2*I*H/2 + 2*I*H/32 + H*I/2 + H*I/32
    assert bench.bytes_per_expert(7168, 2048, False) == 23_396_352


def test_committed_traffic_summary_is_read():
    E, K, H, I, limit, biases, dT, pT = bench.WORKLOADS["gptoss120b"]
    dec, pre, src = bench.measured_traffic("gptoss120b", dT, pT)
    assert src and (ROOT / src).exists()
    # rocprofv3 FETCH + WRITE of one decode gate_up launch: within a few percent above the
    # algorithmic bytes of the ~109 experts a 64-token step touches
    algo = 109 * bench.gate_up_bytes_per_expert(H, I, biases)
    assert algo * 0.97 < dec < algo * 1.10
    assert pre is not None and pre > 128 * bench.gate_up_bytes_per_expert(H, I, biases)
    assert bench.measured_traffic("gptoss120b", dT + 1, pT)[0] is None
