"""PPO training on the GPU against the oracle (model/ppo.h:906-943): one
minibatch and short multi-minibatch runs on the GPU's own rollout, comparing
the recomputed head (1e-4), the Adam first moment (a scaled copy of the
clipped gradient), LossStats and the post-Adam weights (1e-3)."""
import numpy as np
import pytest

from parity import ENVS, THREADS, TOL_HEAD, TOL_TRAIN, assert_close

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


def group_errors(pv, a, b):
    """Relative L2 error per parameter group (canonical layout offsets)."""
    L, E, H, HD = pv.layers, pv.embed, pv.hidden, pv.head_dim
    groups = {"in_w": (pv.off_in_w, pv.obs_dim * E), "in_b": (pv.off_in_b, E), "head": (pv.off_head, E * HD)}
    for l in range(L + 1):
        groups[f"ln{l}_gamma"] = (pv.off_ln_gamma[l], E)
        groups[f"ln{l}_beta"] = (pv.off_ln_beta[l], E)
    for l in range(L):
        groups[f"up{l}"] = (pv.off_up[l], E * H)
        groups[f"down{l}"] = (pv.off_down[l], H * E)
    if pv.continuous:
        groups["log_std"] = (pv.off_log_std, pv.act_dim)
    out = {}
    for k, (o, c) in groups.items():
        x, y = a[o:o + c].astype(np.float64), b[o:o + c].astype(np.float64)
        out[k] = float(np.linalg.norm(x - y) / max(np.linalg.norm(y), 1e-30))
    return out


def relu_flip_units(pv, m_gpu, m_orc):
    """A hidden pre-activation within ~1e-6 of zero can fall on either side of
    the ReLU under a different fp32 summation order; that unit's gradient path
    then switches on or off for that row. Its signature: one hidden column of an
    up matrix holds almost all of that matrix's difference, and the difference
    spreads from there into the layers below (never into the blocks above or
    the head). Returns the blocks showing it."""
    flips = []
    for l in range(pv.layers):
        o, c = pv.off_up[l], pv.embed * pv.hidden
        d = (m_gpu[o:o + c].astype(np.float64) - m_orc[o:o + c]).reshape(pv.embed, pv.hidden)
        col = (d ** 2).sum(0)
        share = col.max() / max(col.sum(), 1e-300)
        print(f"up{l}: worst hidden column {col.argmax()} holds {share:.3f} of the squared difference")
        if share > 0.9:
            flips.append(l)
    return flips


def check_moment(pv, m_gpu, m_orc, params, rows, hp):
    """The GPU's first Adam moment against the oracle's (1e-3 relative L2 per
    parameter group) and both against a float64 gradient: the GPU must be as
    close to float64 as the oracle is. Where the ReLU-flip signature explains a
    difference, the groups it reaches (the flipped block's up matrix and
    everything below it) are held to the float64 reference at 1e-2 instead, and
    every group above it stays at the strict bar."""
    m64 = float64_moment(pv, params, rows, hp)
    e_pair, e_gpu, e_orc = group_errors(pv, m_gpu, m_orc), group_errors(pv, m_gpu, m64), group_errors(pv, m_orc, m64)
    print("gpu vs oracle:", e_pair)
    print("float64 error per group, gpu:", e_gpu, "oracle:", e_orc)
    flips = relu_flip_units(pv, m_gpu, m_orc) if max(e_pair.values()) >= 1e-3 else []
    top = max(flips) if flips else -1  # the highest flipped block

    def below(k):  # groups the flip of block `top` reaches
        if k.startswith(("in_", "ln0")):
            return top >= 0
        for l in range(pv.layers):
            if k in (f"up{l}", f"down{l}", f"ln{l + 1}_gamma", f"ln{l + 1}_beta"):
                return (l < top) or (k == f"up{l}" and l == top) or (k.startswith("ln") and l + 1 <= top)
        return False

    for k in e_gpu:
        if below(k):
            assert e_gpu[k] < 1e-2, (k, e_gpu[k])
        else:
            assert e_pair[k] < 1e-3, (k, e_pair[k])
            assert e_gpu[k] <= 4 * e_orc[k] + 2e-5, (k, e_gpu[k], e_orc[k])


def float64_moment(pv, params, rows, hp):
    """0.1 x the clipped gradient of the minibatch loss in float64, from the torch
    restatement that generates the golden fixtures (tests/golden/make_golden.py)."""
    import torch

    from golden import make_golden as mk

    O, A, E, H, L, cont = pv.obs_dim, pv.act_dim, pv.embed, pv.hidden, pv.layers, bool(pv.continuous)
    obs, acts, adv, ret, old = rows
    t = mk.torch_params(params, O, A, E, H, L, cont)
    head = mk.forward(t, torch.tensor(obs, dtype=torch.float64), E, L)
    act_t = torch.tensor(acts, dtype=torch.float64 if cont else torch.int64)
    f64 = lambda x: torch.tensor(x, dtype=torch.float64)
    loss, _, _ = mk.ppo_loss(head, A, cont, t, act_t, f64(adv), f64(ret), f64(old), hp.clip, hp.value_coef,
                             hp.entropy_coef)
    loss.backward()
    off, count = mk.layout(O, A, E, H, L, cont)
    g = np.zeros(count)
    for k, v in t.items():
        g[off[k]:off[k] + v.numel()] = v.grad.numpy().ravel()
    norm = np.linalg.norm(g)
    scale = hp.max_grad_norm / (norm + 1e-6) if norm > hp.max_grad_norm else 1.0
    return 0.1 * g * scale


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
    ("cartpole", 1024, 2, 512, 1, 5, 2),      # five blocks
    ("cartpole", 1024, 2, 512, 0, 8, 1),      # the most blocks (MG_MAX_LAYERS), hidden 128
    ("cartpole", 1024, 2, 512, 1, 2, 8),      # the widest hidden layer (scale 8: 1024)
    ("cartpole", 1024, 2, 512, 1, 1, 2),      # one block, hidden 256
])
def test_one_minibatch(mg, orc, env, n, T, B, block, layers, scale):
    gym, model, d = setup(mg, orc, env, n, T, B, layers=layers, scale=scale)
    s = model.download_slots()
    p0 = model.params()
    hp = orc.hparams()
    model.train_block(block)
    p1 = model.params()
    m1, v1, step = model.adam_state()
    assert step == 1
    P, M, V = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    st, grad, head = orc.train_minibatch(d, hp, P, M, V, 1, *block_rows(s, n, B, block), threads=THREADS)
    assert_close(model.head(), head, TOL_HEAD, "recomputed head")
    check_moment(model.pv, m1, M, p0, block_rows(s, n, B, block), hp)
    assert_close(p1, P, TOL_TRAIN, "post-Adam weights")
    got, want = np.array(model.last_stats().as_tuple()), np.array(st.as_tuple())
    assert_close(got[[0, 1, 2, 3, 5]], want[[0, 1, 2, 3, 5]], TOL_TRAIN, "LossStats")
    assert abs(got[4] - want[4]) * B <= 2.0 + 1e-3, (got[4], want[4])
    assert np.all(np.isfinite(p1))


@pytest.mark.parametrize("env", ["cartpole", "cartpole_continuous", "cartpole_continuous_clamp", "voxelnav"])
def test_train_epochs(mg, orc, env):
    """train(2) over 2 slots x 2 blocks: the block order and every minibatch's
    LossStats match the oracle's train loop; weights stay within 1e-3."""
    n, T, B = 1024, 2, 512
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


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_full_size_iteration_properties(mg, precision):
    """The benchmarked full-PPO configuration at full size (262144 envs, T = 32,
    4 epochs of 4096-row minibatches = 8192 Adam steps): every epoch visits each
    block once, every minibatch's LossStats are finite and in range, the weights
    stay finite, and a second model from the same seed reproduces the run bit
    for bit (every reduction has a fixed order; in bf16 mode the weight
    gradients come from the fused kernel)."""
    n, T, epochs = 262144, 32, 4
    blocks = T * n // 4096

    def run():
        gym = mg.Gym("rollout_cartpole", n, 0)
        model = mg.PPOModel(gym, horizon=T, precision=precision)
        model.collect()
        model.train(epochs)
        return model

    a = run()
    order = a.last_order()
    assert order.size == epochs * blocks
    for e in range(epochs):
        assert np.array_equal(np.sort(order[e * blocks:(e + 1) * blocks]), np.arange(blocks)), f"epoch {e}"
    st = a.train_stats()
    assert st.shape == (epochs * blocks, 6)
    assert np.isfinite(st).all()
    assert (st[:, 4] >= 0).all() and (st[:, 4] <= 1).all()      # clip fraction
    assert (st[:, 1] >= 0).all() and (st[:, 5] >= 0).all()      # value loss, grad norm
    assert (st[:, 2] >= 0).all() and (st[:, 2] <= np.log(2) + 1e-6).all()  # categorical(2) entropy
    pa = a.params()
    assert np.isfinite(pa).all()
    b = run()
    assert np.array_equal(b.params().view(np.uint32), pa.view(np.uint32)), "rerun differs"
    assert np.array_equal(b.train_stats().view(np.uint32), st.view(np.uint32)), "rerun LossStats differ"
