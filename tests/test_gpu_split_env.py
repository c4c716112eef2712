"""The split observation (OBS_SPLIT in include/mg/env.h) against step(): the
test-only ray-casting envs of tests/envs/raygrid.h, each built twice in the
test env library, the second declaring its rays as independent parts. For
RayGrid (a 272-byte State) the kernels that spread the parts over a workgroup
(rollout_split_kernel; collect with the states in LDS or, at two workgroups per
CU, in device memory) must give the same bits as the plain env's kernels, which
call step() per env lane. RayField's 20-byte State lives in the env lane's
registers, so every kernel must call step() for it despite the split
declaration, at every collect layout."""
import ctypes
import os

import numpy as np
import pytest

from parity import assert_bit_exact

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "envs", "build", "libmg_test_envs.so")
PLAIN, SPLIT = "rollout_test_raygrid", "rollout_test_raygrid_split"
PAIRS = {"raygrid": (PLAIN, SPLIT), "rayfield": ("rollout_test_rayfield", "rollout_test_rayfield_split")}


@pytest.fixture(scope="module")
def envs(mg):
    assert os.path.exists(LIB), f"{LIB} missing: run __graft_entry__.build()"
    ctypes.CDLL(LIB)  # its static initialisers register the envs with the loaded library
    assert {k for p in PAIRS.values() for k in p} <= set(mg.env_names())
    return mg


def same_gym(a, b, what):
    assert_bit_exact(b.state(), a.state(), f"{what} state")
    assert_bit_exact(b.rng(), a.rng(), f"{what} rng")
    assert_bit_exact(b.done(), a.done(), f"{what} done")


@pytest.mark.parametrize("pair", ["raygrid", "rayfield"])
@pytest.mark.parametrize("n", [1001, 4099, 33001])  # 2 envs per workgroup (one wave), the last one partial
def test_split_rollout_matches_step(envs, n, pair):
    mg = envs
    plain, split = PAIRS[pair]
    a, b = mg.Gym(plain, n, 3), mg.Gym(split, n, 3)
    same_gym(a, b, "init")
    ended = np.zeros(n, bool)
    for rep in range(3):  # 150 steps: past the 100-step cap, so every env resets
        sa = a.download_slots(a.rollout_random(50), 50)
        sb = b.download_slots(b.rollout_random(50), 50)
        for x, y, what in zip(sa, sb, ("actions", "obs", "reward", "done")):
            assert_bit_exact(y, x, f"n={n} rep {rep} {what}")
        ended |= sa[3].any(axis=0).astype(bool)
        same_gym(a, b, f"n={n} rep {rep}")
    assert ended.all()


@pytest.mark.parametrize("pair", ["raygrid", "rayfield"])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("n", [
    1024,    # 16-row tiles, states in LDS for both
    8192,    # 32-row tiles, 256 workgroups: states in LDS for both
    16384,   # 32-row tiles, 512 workgroups: the split env's states in device memory, two workgroups per CU
    32768,   # 64-row tiles: both envs' states in device memory
])
def test_split_collect_matches_step(envs, n, bf16, pair):
    """RayField at 16384 and 32768 envs: the two-workgroup layout whose split
    parts would read the states from device memory, where a register-held
    State is not written until the collect ends."""
    mg = envs
    runs = []
    for kernel in PAIRS[pair]:
        g = mg.Gym(kernel, n, 1)
        runs.append((g, mg.PPOModel(g, horizon=4, precision="bf16" if bf16 else "fp32")))
    assert_bit_exact(runs[1][1].params(), runs[0][1].params(), "initial parameters")
    for c in range(3):  # the first call's extra step, then obs[T] -> obs[0]
        outs = []
        for g, m in runs:
            m.collect()
            outs.append((m.download_slots(), m.head()))
        (sa, ha), (sb, hb) = outs
        for key in ("obs", "actions", "logp", "value", "reward", "done", "adv", "ret"):
            assert_bit_exact(sb[key], sa[key], f"n={n} collect {c} {key}")
        assert_bit_exact(hb, ha, f"n={n} collect {c} bootstrap head")
        same_gym(runs[0][0], runs[1][0], f"n={n} collect {c}")
