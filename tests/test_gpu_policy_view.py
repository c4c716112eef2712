"""The policy view (mg_ppo_policy) as a caller's own collect loop uses it: an
env's fused collect kernel launched through its descriptor
(mg_env_desc.collect) with the view. A train step rewrites only the
fragment-tiled copies that the next minibatch reads, so after training the
copy that collect reads (frag_fwd32) lags the parameters until mg_ppo_policy
re-derives it; a view taken after that call, or one held from before training
(the pointers never change), collects exactly what mg_ppo_collect collects
from the same env state."""
import ctypes as C

import numpy as np
import pytest

from parity import assert_bit_exact

pytestmark = pytest.mark.gpu


def collect_with_view(mg, gym, pv, T, last_obs):
    """One collect (not the first) of gym's envs into fresh slot buffers with
    view pv, launched through the env's descriptor; last_obs is the previous
    collect's obs slot T, where this one starts. Returns the slots and the
    bootstrap head."""
    n, O, HD = gym.n, gym.obs_dim, pv.head_dim
    bufs = {
        "obs": mg.DeviceBuffer((T + 1) * n * O * 4),
        "actions": mg.DeviceBuffer(T * n * gym.action_bytes),
        "logp": mg.DeviceBuffer(T * n * 4),
        "value": mg.DeviceBuffer(T * n * 4),
        "reward": mg.DeviceBuffer(T * n * 4),
        "done": mg.DeviceBuffer(T * n),
        "head": mg.DeviceBuffer(n * HD * 4),
    }
    mg.h2d(bufs["obs"].ptr + T * n * O * 4, last_obs)
    a = mg.CollectArgs()
    a.stream, a.policy, a.n, a.horizon, a.first = gym.buf.stream, pv, n, T, 0
    a.state, a.rng, a.done = gym.buf.state, gym.buf.rng, gym.buf.done
    a.obs_slots, a.action_slots, a.logp_slots = bufs["obs"].ptr, bufs["actions"].ptr, bufs["logp"].ptr
    a.value_slots, a.reward_slots, a.done_slots = bufs["value"].ptr, bufs["reward"].ptr, bufs["done"].ptr
    a.head_out = bufs["head"].ptr
    desc = mg.env_desc(gym.kernel)
    rc = mg.COLLECT_FN(desc.collect)(C.byref(a))
    assert rc == 0, rc
    gym.sync()
    return {
        "obs": bufs["obs"].download(np.float32, (T + 1, n, O)),
        "actions": bufs["actions"].download(gym.action_dtype, gym.action_shape(T, n)),
        "logp": bufs["logp"].download(np.float32, (T, n)),
        "value": bufs["value"].download(np.float32, (T, n)),
        "reward": bufs["reward"].download(np.float32, (T, n)),
        "done": bufs["done"].download(np.uint8, (T, n)),
    }, bufs["head"].download(np.float32, (n, HD))


@pytest.mark.parametrize("kernel,n", [("rollout_cartpole", 16384),                # 32-row tiles
                                      ("rollout_cartpole_continuous", 65536)])   # 64-row tiles
def test_view_collect_after_training(mg, kernel, n):
    T = 4
    gym = mg.Gym(kernel, n, 2)
    model = mg.PPOModel(gym, horizon=T, seed=2)
    held = model.pv  # the view taken at creation
    model.collect()
    model.train(1)
    count = model.pv.count
    frag_before = mg.d2h(held.frag_fwd32, np.float32, (count,))
    pv = model.policy()  # re-derives the copies that training left behind
    frag_after = mg.d2h(pv.frag_fwd32, np.float32, (count,))
    for f in ("params", "frag_fwd32", "frag_fwd16", "frag_bwd16"):
        assert getattr(pv, f) == getattr(held, f), f"{f} moved"
    assert not np.array_equal(frag_before, frag_after), "training left frag_fwd32 current: the test shows nothing"
    # the same env state for both collects
    state, rng, done = gym.state(), gym.rng(), gym.done()
    got, got_head = collect_with_view(mg, gym, held, T, model.download_slots()["obs"][T])
    mg.h2d(gym.buf.state, state)
    mg.h2d(gym.buf.rng, rng)
    mg.h2d(gym.buf.done, done)
    model.collect()
    want = model.download_slots()
    for key in got:
        assert_bit_exact(got[key], want[key], f"{kernel} {key}")
    assert_bit_exact(got_head, model.head(), f"{kernel} bootstrap head")
