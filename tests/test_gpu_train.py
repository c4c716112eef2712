"""PPO training on the GPU against the oracle (model/ppo.h:906-943): one
minibatch and short multi-minibatch runs on the GPU's own rollout. A single
minibatch is held exactly (parity.check_minibatch): the oracle replays the
GPU's ReLU decisions, then the recomputed head (1e-4), both Adam moments of
every parameter group (1e-3), LossStats and the post-Adam weights (1e-3)."""
import numpy as np
import pytest

from parity import ENVS, THREADS, TOL_TRAIN, assert_close, check_minibatch, group_errors  # noqa: F401

pytestmark = pytest.mark.gpu


def setup(mg, orc, env, n, T, B, seed=0, layers=2, scale=4):
    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, n, seed)
    model = mg.PPOModel(gym, scale=scale, layers=layers, horizon=T, seed=seed, minibatch=B)
    d = orc.dims(eid, hidden=128 * scale, layers=layers)
    model.collect()
    return gym, model, d


def block_rows(s, n, B, block):
    per = n // B
    t, r0 = block // per, (block % per) * B
    sl = slice(r0, r0 + B)
    return (s["obs"][t, sl], s["actions"][t, sl], s["adv"][t, sl], s["ret"][t, sl], s["logp"][t, sl])


@pytest.mark.parametrize("env,n,T,B,block,layers,scale", [
    ("cartpole", 4096, 2, 4096, 1, 2, 4),
    ("cartpole", 2048, 2, 512, 5, 2, 4),
    ("cartpole", 1280, 2, 320, 3, 2, 4),      # minibatch not a multiple of 128
    ("cartpole", 64, 2, 64, 1, 2, 4),         # the smallest minibatch and env count
    ("cartpole_continuous", 2048, 2, 1024, 2, 2, 4),
    ("cartpole_continuous_clamp", 2048, 2, 1024, 0, 2, 4),
    ("voxelnav16", 1024, 2, 512, 1, 2, 4),
    ("voxelnav", 1024, 2, 512, 1, 2, 4),
    ("cartpole", 1024, 2, 512, 2, 3, 2),      # hidden 256, three blocks
    ("cartpole", 1024, 2, 512, 1, 4, 2),      # four blocks: the most the 8-wave split row pass takes
    ("cartpole", 1024, 2, 512, 1, 5, 2),      # five blocks: the 4-wave split row pass
    ("cartpole", 1024, 2, 512, 0, 8, 1),      # the most blocks (MG_MAX_LAYERS), hidden 128
    ("cartpole", 1024, 2, 512, 1, 2, 8),      # the widest hidden layer (scale 8: 1024)
    ("cartpole", 1024, 2, 512, 1, 1, 2),      # one block, hidden 256
])
def test_one_minibatch(mg, orc, env, n, T, B, block, layers, scale):
    gym, model, d = setup(mg, orc, env, n, T, B, layers=layers, scale=scale)
    s = model.download_slots()
    p0 = model.params()
    model.train_block(block)
    check_minibatch(model, orc, d, orc.hparams(), p0, block_rows(s, n, B, block), B)


@pytest.mark.parametrize("env,n,B", [(e, 1024, 512) for e in ("cartpole", "cartpole_continuous",
                                                                 "cartpole_continuous_clamp", "voxelnav16", "voxelnav")]
                         + [("cartpole", 8192, 4096), ("cartpole_continuous", 8192, 4096)])  # the benchmark minibatch
def test_train_epochs(mg, orc, env, n, B):
    """train(2) over 2 slots x n / B blocks (8 Adam steps): the block order and
    every minibatch's LossStats match the oracle's train loop; weights stay
    within 1e-3. At B = 4096 each step runs the benchmark's minibatch shape
    (256 row tiles, 256 weight-gradient tiles) on rows the earlier steps'
    weights produced."""
    T = 2
    eid, _ = ENVS[env]
    gym, model, d = setup(mg, orc, env, n, T, B, seed=7)
    s = model.download_slots()
    p0 = model.params()
    model.train(2)
    stats = model.train_stats()
    order = model.last_order()
    P, M, V = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    import ctypes as C

    step = C.c_uint32(0)
    shuf = C.c_uint64(0)
    orc.lib().orc_shuffle_state_init(7, C.byref(shuf))
    blocks = T * (n // B)
    order_state = np.arange(blocks, dtype=np.uint32)
    ost = (orc.Stats * (2 * blocks))()
    acts = np.ascontiguousarray(s["actions"])
    orc.lib().orc_train(C.byref(d), C.byref(orc.hparams()), orc.ptr(P), orc.ptr(M), orc.ptr(V), C.byref(step),
                        C.byref(shuf), n, T, B, 2, orc.ptr(np.ascontiguousarray(s["obs"])), orc.ptr(acts),
                        orc.ptr(np.ascontiguousarray(s["adv"])), orc.ptr(np.ascontiguousarray(s["ret"])),
                        orc.ptr(np.ascontiguousarray(s["logp"])), ost, orc.ptr(order_state), THREADS)
    # replay the oracle's order
    shuf2 = C.c_uint64(0)
    orc.lib().orc_shuffle_state_init(7, C.byref(shuf2))
    o = np.arange(blocks, dtype=np.uint32)
    want = []
    for _ in range(2):
        orc.lib().orc_shuffle_blocks(C.byref(shuf2), orc.ptr(o), blocks)
        want += list(o)
    assert list(order) == want
    assert step.value == 2 * blocks
    ostats = np.array([ost[i].as_tuple() for i in range(2 * blocks)], np.float32)
    # clip_frac counts rows with |ratio - 1| > clip: a row sitting on the clip
    # boundary may land on either side, so it is compared in whole rows
    cols = [0, 1, 2, 3, 5]
    assert_close(stats[:, cols], ostats[:, cols], TOL_TRAIN, "per-minibatch LossStats")
    assert np.all(np.abs(stats[:, 4] - ostats[:, 4]) * B <= 2.0 + 1e-3), (stats[:, 4], ostats[:, 4])
    assert_close(model.params(), P, TOL_TRAIN, "weights after 2 epochs")


def test_full_loop_learns(mg):
    """A short CartPole run on the real path improves the mean episode length."""
    gym = mg.Gym("rollout_cartpole", 4096, 0)
    model = mg.PPOModel(gym, horizon=32)
    lens = []
    for it in range(12):
        model.collect()
        d = model.download_slots()["done"]
        lens.append(d.size / max(1, d.sum()))
        model.train(4)
        st = model.last_stats()
        assert np.all(np.isfinite(st.as_tuple()))
    assert np.mean(lens[-3:]) > 1.5 * np.mean(lens[:3]), lens


@pytest.mark.parametrize("env,n,precision", [
    ("cartpole", 262144, "fp32"),             # config 3
    ("cartpole", 262144, "bf16"),
    ("cartpole_continuous", 65536, "fp32"),   # config 4
    ("cartpole_continuous", 262144, "fp32"),
    ("voxelnav16", 262144, "fp32"),           # config 5, full PPO
])
def test_full_size_iteration_properties(mg, env, n, precision):
    """A benchmarked full-PPO configuration at full size (T = 32, 4 epochs of
    4096-row minibatches: 8192 Adam steps at 262144 envs): every epoch visits
    each block once, every minibatch's LossStats are finite and in range, the
    weights stay finite, and a second model from the same seed reproduces the
    run bit for bit (every reduction has a fixed order; in bf16 mode the weight
    gradients come from the fused kernel)."""
    T, epochs = 32, 4
    blocks = T * n // 4096
    eid, kernel = ENVS[env]

    def run():
        gym = mg.Gym(kernel, n, 0)
        model = mg.PPOModel(gym, horizon=T, precision=precision)
        model.collect()
        model.train(epochs)
        return gym, model

    gym, a = run()
    order = a.last_order()
    assert order.size == epochs * blocks
    for e in range(epochs):
        assert np.array_equal(np.sort(order[e * blocks:(e + 1) * blocks]), np.arange(blocks)), f"epoch {e}"
    st = a.train_stats()
    assert st.shape == (epochs * blocks, 6)
    assert np.isfinite(st).all()
    assert (st[:, 4] >= 0).all() and (st[:, 4] <= 1).all()      # clip fraction
    assert (st[:, 1] >= 0).all() and (st[:, 5] >= 0).all()      # value loss, grad norm
    if gym.continuous:  # Gaussian entropy sum_k (log_std_k + ln(2 pi) / 2 + 1 / 2) of the step's log_std
        assert (np.abs(st[:, 2] - (0.5 * np.log(2 * np.pi) + 0.5)) < 0.1).all()
    else:  # categorical(A) entropy
        assert (st[:, 2] >= 0).all() and (st[:, 2] <= np.log(gym.act_dim) + 1e-6).all()
    pa = a.params()
    assert np.isfinite(pa).all()
    del a, gym
    _, b = run()
    assert np.array_equal(b.params().view(np.uint32), pa.view(np.uint32)), "rerun differs"
    assert np.array_equal(b.train_stats().view(np.uint32), st.view(np.uint32)), "rerun LossStats differ"
