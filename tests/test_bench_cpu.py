"""bench.py's command-line contract, checked without a GPU: more than one GPU is refused
with a message and exit status 2 before anything touches a device, and the algorithmic
counts the roofline uses match the closed forms of the config-2 workload."""
import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
    assert proc.stdout == ""


def test_config2_counts():
    import bench

    flops, bytes_ = bench.c2_counts()
    tokens, dk, dv, C = 64 * 2048, 128, 128, 64
    # FLOPs per token 2C(d_k + d_v) + 4 d_k d_v (dense-chunk convention)
    assert flops == tokens * (2 * C * (dk + dv) + 4 * dk * dv) == 12_884_901_888
    # q, k, v in bf16, hidden out in bf16, the fp32 initial state and 32 fp32 snapshots per sequence
    expect = tokens * (2 * dk + dv) * 2 + tokens * dv * 2 + 64 * dv * dk * 4 + 64 * 32 * dv * dk * 4
    assert bytes_ == expect == 272_629_760
