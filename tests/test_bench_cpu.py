"""bench.py's host-side contract (CPU): the multi-GPU refusal, the no-GPU exit, and the
per-launch HBM traffic each roofline object reads from the committed counter profiles."""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _bench(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused_with_a_reason():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_gpu_exits_with_a_message():
    r = _bench("--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "needs a ROCm GPU" in r.stderr


@pytest.mark.parametrize("profile,key", [
    ("decode_c3_traffic.md", ""),                       # the headline roofline
    ("decode_c2_traffic.md", ""),                       # c2_decode_roofline
    ("verify_c4_traffic.md", "c4_verify"),              # c4_verify_roofline
    ("byte_movers_c4_c5_traffic.md", "c5_gather"),      # c5_gather_roofline
    ("byte_movers_c4_c5_traffic.md", "c5_scatter"),     # c5_scatter_roofline
    ("byte_movers_c4_c5_traffic.md", "c5_map"),         # c5_map_roofline
])
def test_every_roofline_finds_its_counter_traffic(profile, key):
    sys.path.insert(0, str(ROOT))
    import bench
    traffic = bench._traffic_per_launch(profile, key)
    assert isinstance(traffic, int) and traffic > 0, (profile, key)
    assert str(traffic) in (ROOT / "profiles" / profile).read_text()
