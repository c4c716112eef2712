"""bench.py's contract on the CPU: more than one GPU is refused with a message
before anything touches a device, and the figures the CPU baseline reports
about the host (threads used, cores available) are sane."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, (r.returncode, r.stdout, r.stderr)
    assert "one MI355X" in r.stderr and "--gpus must be 1" in r.stderr
    assert r.stdout == ""  # no JSON line for a configuration that was not measured


def test_host_core_figures():
    sys.path.insert(0, ROOT)
    import bench

    cores, usable = bench.host_cores()
    threads = bench.cpu_threads()
    assert cores >= 1 and 1 <= usable <= cores
    assert 1 <= threads <= min(usable, 16)
