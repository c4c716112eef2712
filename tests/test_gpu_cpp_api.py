"""The header-only C++ API (Gym<Env>, PPOModel<Env>) and a user-defined env
registered with MG_DEFINE_ENV, run as compiled programs on the GPU."""
import math
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


def test_continuous_example_runs_and_learns():
    """The reference's CartPoleContinuous loop (examples/CartPoleContinuous/
    main.cpp:23-46, here examples/cartpole_continuous.cpp): its printed lines
    are consistent with each other and the episodes get longer. The entropy a
    minibatch reports is that of its Gaussian head, log std + ln(2 pi) / 2 +
    1 / 2, one Adam step before the std printed beside it; the approximate KL
    of the last minibatch stays small (measured up to 0.06 after 4 epochs; a
    broken loss or gradient gives values of order 1 or NaN)."""
    p = run("cartpole_continuous")
    assert p.returncode == 0
    rows = []
    for line in p.stdout.splitlines():
        if line.startswith("iter"):
            t = line.split()
            rows.append((int(t[1]), float(t[3]), float(t[5]), float(t[7]), float(t[9])))
    assert [r[0] for r in rows] == [0, 10, 20, 30, 40, 50, 59]
    for it, length, std, ent, kl in rows:
        assert length > 0 and std > 0
        assert abs(ent - (math.log(std) + 0.5 * math.log(2 * math.pi) + 0.5)) < 3e-3, (it, std, ent)
        assert abs(kl) < 0.2, (it, kl)
    assert max(r[1] for r in rows[-2:]) > 2 * rows[0][1], rows
