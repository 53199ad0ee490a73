"""bench.py's host-side parts (no GPU): the one-GPU refusal and the roofline
inputs it reads from the committed profiles."""

from __future__ import annotations

import importlib.util
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "multi-GPU" in r.stderr and r.stdout == ""


def test_every_step_kernel_has_committed_traffic_at_config2():
    b = _bench()
    status = {"selected": [1442, 1436, 1439, 1436], "scanned": [0, 0, 0, 0],
              "pool": [40627, 40351, 40792, 40693], "u1": [6047, 6027, 6055, 6052]}
    p = SimpleNamespace(sink=128, local=256)
    nbytes = b.kernel_bytes(status, p, 8192)
    assert list(nbytes) == ["front", "select", "pool", "top1600", "union_score", "top256",
                            "top100_sdpa"]
    for name, algo in nbytes.items():
        traffic = b.measured_traffic(name, "cfg2")
        assert traffic is not None, name
        assert algo > 0 and traffic > 0, name
    assert b.measured_traffic("no_such_kernel", "cfg2") is None
    assert b.measured_traffic("top1600", "no_such_config") is None


def test_top1600_bytes_per_launch_at_config2():
    """The dominant kernel's algorithmic bytes: 2 B per (pool key, head) in
    plus a member bitmap of ceil(n / 64) 8-byte words per (group, head) out;
    at the config-2 pool sizes of the bench line that is 1,380,984 B."""
    b = _bench()
    pools = [40627, 40351, 40792, 40693]
    status = {"selected": [0] * 4, "scanned": [0] * 4, "pool": pools, "u1": [0] * 4}
    got = b.kernel_bytes(status, SimpleNamespace(sink=128, local=256), 8192)["top1600"]
    assert got == sum(pools) * 4 * 2 + 4 * sum((n + 63) // 64 * 8 for n in pools)
    assert got == 1_380_984
