"""The header-only C++ API (Gym<Env>, PPOModel<Env>) and a user-defined env
registered with MG_DEFINE_ENV, run as compiled programs on the GPU."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BUILD = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "examples", "build")


def run(prog, *args, timeout=240):
    path = os.path.join(BUILD, prog)
    assert os.path.exists(path), f"{path} missing: run __graft_entry__.build()"
    p = subprocess.run([path, *args], capture_output=True, text=True, timeout=timeout)
    print(p.stdout, p.stderr)
    return p


def test_api_check():
    p = run("api_check")
    assert p.returncode == 0 and "api_check ok" in p.stdout


def test_user_defined_env_trains():
    p = run("custom_env")
    assert p.returncode == 0, p.stdout


def test_reference_training_loop_runs():
    p = run("cartpole")
    assert p.returncode == 0
    lines = [l for l in p.stdout.splitlines() if l.startswith("iter")]
    assert len(lines) == 4


def test_voxelnav_learns():
    """The reference's VoxelNav loop (examples/VoxelNav/main.cpp): the success
    rate (episodes ending with reward > 5) rises well above its start."""
    p = run("voxelnav", "150", timeout=300)
    assert p.returncode == 0
    rates = [float(l.split()[3]) for l in p.stdout.splitlines() if l.startswith("iter")]
    assert len(rates) >= 10
    assert max(rates[-3:]) > max(0.3, 3 * rates[0]), rates
