"""rollout<Env> on the GPU against the oracle: RNG streams, env state, resets,
done flags, observations and rewards must be bit-exact (rollout.h:31-54)."""
import numpy as np
import pytest

from parity import ENVS, THREADS, assert_bit_exact

pytestmark = pytest.mark.gpu


def compare_gym(gym, g, what):
    assert_bit_exact(gym.state(), g.state, f"{what} state")
    assert_bit_exact(gym.rng(), g.rng, f"{what} rng")
    assert_bit_exact(gym.done(), g.done, f"{what} done")


@pytest.mark.parametrize("env,n,steps,seed", [
    ("cartpole", 4096, 32, 0),
    ("cartpole", 1000, 600, 3),           # ragged n; long enough for truncation at 500
    ("cartpole_continuous", 2048, 64, 0),
    ("cartpole_continuous_clamp", 2048, 64, 1),
    ("voxelnav16", 512, 300, 0),          # past the 256-step cap
    ("voxelnav", 512, 300, 2),            # past the 250-step cap
])
def test_random_rollout_bit_exact(mg, orc, env, n, steps, seed):
    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, n, seed)
    g = orc.GymState(eid, n, seed)
    compare_gym(gym, g, "init")
    for rep in range(2):  # state carries over between launches
        bufs = gym.rollout_random(steps)
        acts, obs, rew, dn = gym.download_slots(bufs, steps)
        oa, oo, orw, od = orc.rollout(g, steps, random=True, threads=THREADS)
        assert_bit_exact(acts, oa, f"{env} rep {rep} actions")
        assert_bit_exact(obs, oo, f"{env} rep {rep} obs")
        assert_bit_exact(rew, orw, f"{env} rep {rep} reward")
        assert_bit_exact(dn, od, f"{env} rep {rep} done slots")
        compare_gym(gym, g, f"{env} rep {rep}")
    assert dn.any(), "no episode ended: the test does not exercise resets"


@pytest.mark.parametrize("env,n,steps,reps,seed", [
    ("voxelnav", 4101, 40, 7, 4),      # 1 KB states: 2 envs per one-wave workgroup, the last partial
    ("voxelnav", 33001, 20, 13, 5),    # the same at a larger grid
    ("voxelnav16", 4099, 40, 7, 6),    # 4 KB states: 4 per 128-thread workgroup (16.5 KB of LDS), the last partial
    ("voxelnav16", 33001, 20, 13, 7),  # 4 per workgroup at any n, the last partial
])
def test_split_rollout_sizes_bit_exact(mg, orc, env, n, steps, reps, seed):
    """The split-observation rollouts (VoxelNav's ray casts, VoxelNav16's
    neighbourhood cells, spread over each workgroup) at env counts that leave
    the last workgroup partial, run past the 250- and 256-step caps so that
    every env resets at least once (several envs of a workgroup in one step,
    at the first step and at the cap); VoxelNav16 writes its grid back only
    in a launch in which the env reset, which the later launches' observations
    and the final states check."""
    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, n, seed)
    g = orc.GymState(eid, n, seed)
    bufs = None
    ended = np.zeros(n, bool)
    for rep in range(reps):
        bufs = gym.rollout_random(steps, bufs)
        acts, obs, rew, dn = gym.download_slots(bufs, steps)
        oa, oo, orw, od = orc.rollout(g, steps, random=True, threads=THREADS)
        assert_bit_exact(acts, oa, f"rep {rep} actions")
        assert_bit_exact(obs, oo, f"rep {rep} obs")
        assert_bit_exact(rew, orw, f"rep {rep} reward")
        assert_bit_exact(dn, od, f"rep {rep} done slots")
        ended |= dn.any(axis=0).astype(bool)
    compare_gym(gym, g, "end")
    assert ended.all(), f"{int((~ended).sum())} envs never ended"


@pytest.mark.parametrize("env", ["cartpole", "cartpole_continuous", "voxelnav16", "voxelnav"])
def test_given_action_rollout_bit_exact(mg, orc, env):
    """Given actions, launch after launch. The split-observation envs run three
    launches of 100 steps, past their 250- and 256-step caps, so that launches
    in which most envs do not reset (VoxelNav16 then writes back only its
    32-byte header) are followed by ones that read the states back."""
    eid, kernel = ENVS[env]
    split = env in ("voxelnav16", "voxelnav")
    n, steps, reps = 2048, (100 if split else 40), (3 if split else 1)
    gym = mg.Gym(kernel, n, 5)
    g = orc.GymState(eid, n, 5)
    rs = np.random.default_rng(1)
    for rep in range(reps):
        if gym.continuous:
            acts = (rs.standard_normal((steps, n, gym.act_dim)) * 2).astype(np.float32)
        else:
            acts = rs.integers(0, gym.act_dim, (steps, n)).astype(np.int32)
        bufs = gym.rollout_given(steps, acts)
        _, obs, rew, dn = gym.download_slots(bufs, steps)
        _, oo, orw, od = orc.rollout(g, steps, random=False, actions_in=acts, threads=THREADS)
        assert_bit_exact(obs, oo, f"rep {rep} obs")
        assert_bit_exact(rew, orw, f"rep {rep} reward")
        assert_bit_exact(dn, od, f"rep {rep} done")
        compare_gym(gym, g, f"{env} rep {rep}")


def test_gym_run_single_steps(mg, orc):
    """gym.run() (gym.h:110-121): one step from the action buffer into obs/reward."""
    n = 640
    gym = mg.Gym("rollout_cartpole", n, 0)
    g = orc.GymState(0, n, 0)
    rs = np.random.default_rng(2)
    for _ in range(30):
        a = rs.integers(0, 2, n).astype(np.int32)
        gym.set_actions(a)
        gym.run()
        _, oo, orw, _ = orc.rollout(g, 1, random=False, actions_in=a[None], threads=THREADS)
        assert_bit_exact(gym.obs(), oo[0], "obs")
        assert_bit_exact(gym.reward(), orw[0], "reward")
    compare_gym(gym, g, "run")


def test_large_random_rollout_invariants(mg):
    """At the benchmark size, size-independent properties: rewards are 1,
    RNG states never hit the absorbing 0, every done flag matches a threshold
    crossing or the 500-step cap, and obs stay inside the reset box after a reset."""
    n, steps = 262144, 32
    gym = mg.Gym("rollout_cartpole", n, 0)
    bufs = gym.rollout_random(steps)
    acts, obs, rew, dn = gym.download_slots(bufs, steps)
    assert np.all(rew == 1.0)
    assert np.all((acts == 0) | (acts == 1))
    assert np.all(gym.rng() != 0)
    theta_thr = np.float32(12.0 * 2.0 * np.float32(np.pi) / 360.0)
    term = (np.abs(obs[..., 0]) > 2.4) | (np.abs(obs[..., 2]) > theta_thr)
    assert np.array_equal(dn.astype(bool), term)  # no truncation within 32 steps of a fresh start
    # each env's actions are roughly fair coin flips
    assert abs(acts.mean() - 0.5) < 0.01


@pytest.mark.parametrize("env", ["cartpole", "cartpole_continuous", "voxelnav16", "voxelnav"])
def test_step_into_slot_buffers(mg, orc, env):
    """Gym::stepInto (gym.h:94-108, encodeStep): T single steps, step t reading
    slot t of a device action buffer and writing slot t of device obs and
    reward buffers (each at its own offset, as collect writes obs[t + 1]),
    bit for bit against the oracle's given-action rollout; the gym's state,
    RNG and done flags too, and slots beyond the written ones stay untouched."""
    eid, kernel = ENVS[env]
    n, T = 1536, 24
    gym = mg.Gym(kernel, n, 4)
    g = orc.GymState(eid, n, 4)
    rs = np.random.default_rng(8)
    if gym.continuous:
        acts = (rs.standard_normal((T, n, gym.act_dim)) * 2).astype(np.float32)
    else:
        acts = rs.integers(0, gym.act_dim, (T, n)).astype(np.int32)
    abuf = mg.DeviceBuffer.from_array(acts)
    obs_sentinel = np.full((T + 1, n, gym.obs_dim), -7.0, np.float32)
    rew_sentinel = np.full((T + 1, n), -7.0, np.float32)
    obuf = mg.DeviceBuffer.from_array(obs_sentinel)
    rbuf = mg.DeviceBuffer.from_array(rew_sentinel)
    for t in range(T):  # obs into slot t + 1, reward into slot t, as in collect
        gym.step_into(abuf.ptr + t * n * gym.action_bytes, obuf.ptr + (t + 1) * n * gym.obs_dim * 4,
                      rbuf.ptr + t * n * 4)
    gym.sync()
    obs = obuf.download(np.float32, (T + 1, n, gym.obs_dim))
    rew = rbuf.download(np.float32, (T + 1, n))
    _, oo, orw, od = orc.rollout(g, T, random=False, actions_in=acts, threads=THREADS)
    assert_bit_exact(obs[1:], oo, "obs")
    assert_bit_exact(rew[:T], orw, "reward")
    assert np.all(obs[0] == -7.0) and np.all(rew[T] == -7.0), "step_into wrote outside its slots"
    compare_gym(gym, g, env)
    # VoxelNav16 / VoxelNav episodes last up to 256 / 250 steps; the first step's resets still run
    if env not in ("voxelnav16", "voxelnav"):
        assert od.any(), "no episode ended: the test does not exercise resets"
