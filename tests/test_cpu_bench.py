"""bench.py's contract on the CPU: more than one GPU is refused with a message
before anything touches a device, the figures the CPU baseline reports about
the host (threads used, cores available) are sane, and the random rollout's
algorithmic byte count follows the envs' write-back rule."""
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


class _Gym:
    def __init__(self, kernel, obs_dim, action_bytes, state_bytes):
        self.kernel, self.obs_dim, self.action_bytes, self.state_bytes = kernel, obs_dim, action_bytes, state_bytes


def test_rollout_bytes_partial_write_back():
    """The random rollout's algorithmic bytes: an env of STEP_WRITE_BYTES
    writes its header back, and its whole state only in a launch in which it
    reset. With every env reset the count equals the whole-state one, with
    none only the headers are written; the header size matches the env's
    STEP_WRITES declaration."""
    sys.path.insert(0, ROOT)
    import bench

    n, T = 4096, 32
    cart = _Gym("rollout_cartpole", 4, 4, 20)
    assert bench.rollout_bytes(cart, n, T) == n * T * 25 + n * 2 * 25
    assert bench.rollout_bytes(cart, n, T, resets=17) == bench.rollout_bytes(cart, n, T)  # no STEP_WRITES
    vn = _Gym("rollout_voxelnav16", 30, 4, 4128)
    whole = bench.rollout_bytes(vn, n, T)
    assert whole == n * T * 129 + n * 2 * (4128 + 5)
    assert bench.rollout_bytes(vn, n, T, resets=n) == whole
    assert bench.rollout_bytes(vn, n, T, resets=0) == n * T * 129 + n * 10 + n * (4128 + 32)
    assert bench.rollout_bytes(vn, n, T, resets=100) - bench.rollout_bytes(vn, n, T, resets=0) == 100 * (4128 - 32)
    with open(os.path.join(ROOT, "include", "mg", "envs", "voxelnav16.h")) as f:
        src = f.read()
    assert "STEP_WRITES = 8;" in src and bench.STEP_WRITE_BYTES["rollout_voxelnav16"] == 4 * 8
