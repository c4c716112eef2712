"""Pins the CPU oracle before it is trusted as the GPU checker: known answers,
closed forms, textbook equations in double precision, library routines
(torch float64 golden fixtures) and spec invariants. A plausible mistake in the
oracle (a dropped term, a wrong sign or index, a transposed operand, a biased
variance, a missed reset) fails at least one of these."""
import ctypes as C
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


# ---- RNG (rollout.h:9-29, gym.h:57-61) --------------------------------------------

def test_xorshift_known_answers(orc):
    # Marsaglia (2003) xorshift32 with shifts 13/17/5 from state 1
    s = np.array([1], np.uint32)
    assert [orc.lib().orc_rng_next(orc.ptr(s)) for _ in range(3)] == [270369, 67634689, 2647435461]


def test_uniform_is_top_24_bits(orc):
    s = np.array([123456789], np.uint32)
    for _ in range(1000):
        prev = s.copy()
        u = orc.lib().orc_rng_uniform(orc.ptr(s))
        assert u == np.float32(int(s[0]) >> 8) * np.float32(2.0 ** -24)
        assert 0.0 <= u < 1.0
        assert s[0] != prev[0]


def test_rng_int_is_modulo(orc):
    s = np.array([987654321], np.uint32)
    t = s.copy()
    for _ in range(200):
        k = orc.lib().orc_rng_int(orc.ptr(s), 6)
        assert k == orc.lib().orc_rng_next(orc.ptr(t)) % 6


def test_seed_hash(orc):
    n = 4096
    g0 = orc.GymState(orc.CARTPOLE, n, 0)
    i = np.arange(n, dtype=np.uint64)
    assert np.array_equal(g0.rng, ((i * 2654435761 + 1) % 2**32).astype(np.uint32))  # gym.h:57-61
    assert np.all(g0.done == 1) and not g0.actions.any()
    g1 = orc.GymState(orc.CARTPOLE, n, 1)
    assert np.all(g1.rng != 0) and not np.array_equal(g1.rng, g0.rng)


# ---- CartPole (examples/CartPole/cartpole.metal) ----------------------------------------

def cartpole_step_double(x, xd, th, thd, force):
    """Barto, Sutton & Anderson / Gymnasium CartPole-v1 Euler step in double."""
    g, mc, mp, l, tau = 9.8, 1.0, 0.1, 0.5, 0.02
    total, pml = mc + mp, mp * l
    c, s = math.cos(th), math.sin(th)
    temp = (force + pml * thd * thd * s) / total
    thacc = (g * s - c * temp) / (l * (4.0 / 3.0 - mp * c * c / total))
    xacc = temp - pml * thacc * c / total
    return x + tau * xd, xd + tau * xacc, th + tau * thd, thd + tau * thacc


def test_cartpole_first_reset_known_answer(orc):
    state = np.zeros(20, np.uint8)
    rng = np.array([1], np.uint32)  # env 0, seed 0
    orc.lib().orc_env_reset(0, orc.ptr(state), orc.ptr(rng))
    f = state[:16].view(np.float32)
    want = np.array([-0.049993705, -0.048425257, 0.011640407, -0.042838138], np.float32)
    assert np.array_equal(f, want)
    assert rng[0] == 307599695
    assert state[16:].view(np.uint32)[0] == 0


def test_cartpole_step_matches_textbook(orc):
    rs = np.random.default_rng(0)
    for _ in range(2000):
        st = np.zeros(5, np.uint32)
        v = (rs.uniform(-1, 1, 4) * [2.0, 2.0, 0.2, 2.0]).astype(np.float32)
        st[:4] = v.view(np.uint32)
        st[4] = rs.integers(0, 498)
        a = np.array([rs.integers(0, 2)], np.int32)
        obs = np.zeros(4, np.float32)
        r = np.zeros(1, np.float32)
        d = np.zeros(1, np.uint8)
        orc.lib().orc_env_step(0, orc.ptr(st), orc.ptr(a), orc.ptr(obs), orc.ptr(r), orc.ptr(d))
        want = cartpole_step_double(*[float(x) for x in v], 10.0 if a[0] == 1 else -10.0)
        got = st[:4].view(np.float32)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6), (v, got, want)
        assert np.array_equal(obs, got)
        assert r[0] == 1.0
        thr = 12 * 2 * math.pi / 360
        if abs(abs(want[0]) - 2.4) > 1e-5 and abs(abs(want[2]) - thr) > 1e-5:
            assert d[0] == (abs(want[0]) > 2.4 or abs(want[2]) > thr)


def test_cartpole_truncates_at_500(orc):
    st = np.zeros(5, np.uint32)
    st[4] = 499
    a = np.array([1], np.int32)
    obs, r, d = np.zeros(4, np.float32), np.zeros(1, np.float32), np.zeros(1, np.uint8)
    orc.lib().orc_env_step(0, orc.ptr(st), orc.ptr(a), orc.ptr(obs), orc.ptr(r), orc.ptr(d))
    assert d[0] == 1 and st[4] == 500


def test_continuous_force_is_10_tanh(orc):
    for a in (-3.0, -0.4, 0.0, 0.25, 1.0, 5.0):
        st = np.zeros(5, np.uint32)
        st[:4] = np.array([0.0, 0.1, 0.05, -0.1], np.float32).view(np.uint32)
        ref = st.copy()
        act = np.array([a], np.float32)
        obs, r, d = np.zeros(4, np.float32), np.zeros(1, np.float32), np.zeros(1, np.uint8)
        orc.lib().orc_env_step(1, orc.ptr(st), orc.ptr(act), orc.ptr(obs), orc.ptr(r), orc.ptr(d))
        want = cartpole_step_double(0.0, 0.1, 0.05, -0.1, 10.0 * math.tanh(a))
        assert np.allclose(st[:4].view(np.float32), want, rtol=1e-5, atol=1e-6)
        orc.lib().orc_env_step(2, orc.ptr(ref), orc.ptr(act), orc.ptr(obs), orc.ptr(r), orc.ptr(d))
        want = cartpole_step_double(0.0, 0.1, 0.05, -0.1, 10.0 * max(-1.0, min(1.0, a)))
        assert np.allclose(ref[:4].view(np.float32), want, rtol=1e-5, atol=1e-6)


def test_random_rollout_rng_accounting(orc):
    """Per env and step: one action draw, then four reset draws when done was set."""
    n, T = 64, 40
    g = orc.GymState(orc.CARTPOLE, n, 0)
    rng0 = g.rng.copy()
    acts, obs, rew, dn = orc.rollout(g, T, random=True, threads=1)
    resets = 1 + dn[:-1].sum(axis=0).astype(int)  # done starts at 1
    for i in range(n):
        s = np.array([rng0[i]], np.uint32)
        for _ in range(T + 4 * resets[i]):
            orc.lib().orc_rng_next(orc.ptr(s))
        assert s[0] == g.rng[i]


# ---- shared deterministic math (include/mg/math.h) ------------------------------------

def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7fffffff), a)
    b = np.where(b < 0, -(b & 0x7fffffff), b)
    return np.abs(a - b)


@pytest.mark.parametrize("name,fn,lo,hi,tol", [
    ("sinf", np.sin, -40.0, 40.0, 1), ("cosf", np.cos, -40.0, 40.0, 1), ("sinf", np.sin, -1.0, 1.0, 1),
    ("expf", np.exp, -80.0, 80.0, 1), ("expf", np.exp, -2.0, 2.0, 1),
    ("logf", np.log, 1e-30, 1e4, 2), ("tanhf", np.tanh, -12.0, 12.0, 3), ("tanhf", np.tanh, -0.5, 0.5, 3),
])
def test_math_within_stated_ulp_of_libm(orc, name, fn, lo, hi, tol):
    """Float-path accuracy bounds stated in include/mg/math.h's header, against
    numpy's double-precision functions rounded once to float."""
    rs = np.random.default_rng(5)
    if name == "logf":
        xs = np.exp(rs.uniform(np.log(lo), np.log(hi), 20000)).astype(np.float32)
    else:
        xs = rs.uniform(lo, hi, 20000).astype(np.float32)
    xs = np.concatenate([xs, np.array([0.0, 1e-8, -1e-8, 0.2094395, 1.0, 0.5], np.float32)])
    if name == "logf":
        xs = np.abs(xs) + np.float32(1e-30)
    f = getattr(orc.lib(), "orc_" + name)
    got = np.array([f(float(x)) for x in xs], np.float32)
    want = fn(xs.astype(np.float64)).astype(np.float32)
    assert ulp_diff(got, want).max() <= tol


def test_math_edges(orc):
    L = orc.lib()
    assert L.orc_expf(-87.5) == 0.0 and L.orc_expf(-86.9) > 0.0  # no subnormal results
    assert L.orc_expf(0.0) == 1.0 and L.orc_logf(1.0) == 0.0 and L.orc_tanhf(0.0) == 0.0
    assert np.isinf(L.orc_expf(100.0)) and L.orc_tanhf(20.0) == 1.0 and L.orc_tanhf(-20.0) == -1.0
    xs = np.random.default_rng(9).uniform(-20, 20, 2000).astype(np.float32)
    s = np.array([L.orc_sinf(float(x)) for x in xs], np.float64)
    c = np.array([L.orc_cosf(float(x)) for x in xs], np.float64)
    assert np.abs(s * s + c * c - 1.0).max() < 3e-7
    # odd / even symmetry holds exactly on the float path
    for x in (0.3, 1.1, 2.5, 5.9):
        assert L.orc_sinf(-x) == -L.orc_sinf(x) and L.orc_cosf(-x) == L.orc_cosf(x)


# ---- parameters (model/ppo.h:375-423) ------------------------------------------

def test_layout_matches_reference_grouping(orc):
    d = orc.dims(orc.CARTPOLE)
    L = orc.layout(d)
    assert L.float_group == 512 + 128 + 2 * 128 * 3  # in_w, in_b, 3 LayerNorms
    assert L.off_up[0] == L.float_group and L.off_head == L.float_group + 4 * 65536
    assert L.count == L.off_head + 384


def test_splitmix_known_answer(orc):
    s = C.c_uint64(0)
    assert orc.lib().orc_splitmix_next(C.byref(s)) == 0xE220A8397B1DCDAF  # SplitMix64 from state 0


def test_init_distributions(orc):
    d = orc.dims(orc.CARTPOLE)
    L = orc.layout(d)
    p = orc.init_params(d, 0)
    E, H = 128, 512

    def check(seg, std):
        bound = math.sqrt(3.0) * std
        assert np.abs(seg).max() <= bound * (1 + 1e-6)
        n = seg.size  # 4-sigma bounds of the sample statistics
        assert abs(seg.std() - std) < 4 * std / math.sqrt(n)
        assert abs(seg.mean()) < 4 * std / math.sqrt(n)

    check(p[L.off_in_w:L.off_in_w + 4 * E], 1 / math.sqrt(4))
    check(p[L.off_up[1]:L.off_up[1] + E * H], math.sqrt(2 / E))
    check(p[L.off_down[0]:L.off_down[0] + H * E], 1 / math.sqrt(H) / math.sqrt(2))
    head = p[L.off_head:L.off_head + E * 3].reshape(E, 3)
    check(head[:, :2].ravel(), 0.01)
    check(head[:, 2], 1 / math.sqrt(E))
    assert np.all(p[L.off_ln_gamma[2]:L.off_ln_gamma[2] + E] == 1.0)
    assert not p[L.off_ln_beta[0]:L.off_ln_beta[0] + E].any() and not p[L.off_in_b:L.off_in_b + E].any()
    assert np.array_equal(p, orc.init_params(d, 0)) and not np.array_equal(p, orc.init_params(d, 1))


# ---- golden fixtures: torch float64 forward / autograd / clip / Adam ------------------------

def load(name):
    z = np.load(os.path.join(HERE, "golden", name + ".npz"))
    return {k: z[k] for k in z.files}


def fixture_dims(orc, z):
    O, A, E, H, L, cont, B = (int(x) for x in z["dims"])
    return orc.Dims(O, A, E, H, L, cont), B


@pytest.mark.parametrize("name", ["ppo_categorical", "ppo_gaussian", "ppo_voxel_shape"])
def test_forward_vs_torch(orc, name):
    z = load(name)
    d, B = fixture_dims(orc, z)
    head = orc.forward(d, z["params0"], z["obs"], threads=2)
    np.testing.assert_allclose(head, z["head0"], rtol=1e-5, atol=1e-5)


def rel_group_err(got, want):
    return float(np.linalg.norm(got.astype(np.float64) - want) / max(np.linalg.norm(want), 1e-30))


@pytest.mark.parametrize("name", ["ppo_categorical", "ppo_gaussian", "ppo_voxel_shape"])
def test_ppo_minibatch_vs_torch(orc, name):
    """Loss, hand-written backward, grad-norm clip and Adam over several steps
    against torch autograd + clip_grad_norm_ + torch.optim.Adam."""
    z = load(name)
    d, B = fixture_dims(orc, z)
    clip, vc, ec, mgn, gamma, lam, lr = z["hp"]
    hp = orc.hparams(clip=clip, value_coef=vc, entropy_coef=ec, max_grad_norm=mgn, lr=lr)
    P = z["params0"].copy()
    M, V = np.zeros_like(P), np.zeros_like(P)
    steps = sum(1 for k in z if k.startswith("grad"))
    for s in range(steps):
        st, grad, head = orc.train_minibatch(d, hp, P, M, V, s + 1, z["obs"], z["actions"], z["adv"], z["ret"],
                                             z["old_logp"], threads=2)
        np.testing.assert_allclose(head, z[f"head{s}"], rtol=1e-5, atol=1e-5)
        g = z[f"grad{s}"].astype(np.float64)
        assert rel_group_err(grad, g) < 2e-5
        assert np.abs(grad - g).max() <= 1e-4 * np.abs(g).max()
        # Adam moves each weight by about lr * g / (|g| + eps): for a gradient near
        # zero the fp32/fp64 difference of g shows up as a fraction of one step
        np.testing.assert_allclose(P, z[f"params{s + 1}"], rtol=0, atol=0.07 * lr)
        want = z[f"stats{s}"]
        got = np.array(st.as_tuple(), np.float64)
        np.testing.assert_allclose(got[[0, 1, 2, 3, 5]], want[[0, 1, 2, 3, 5]], rtol=1e-5, atol=1e-6)
        assert round(got[4] * B) == round(want[4] * B)  # clip_frac: same rows outside the band
    assert 0 < z["stats0"][4] < 1, "fixture must exercise both clip branches"


# ---- GAE (model/gae.metal:14-36) ------------------------------------------------

def test_gae_closed_form(orc):
    """A_t = sum_l (gamma lambda)^l delta_{t+l}, truncated at the first done, in double."""
    rs = np.random.default_rng(7)
    T, n, A = 7, 300, 2
    reward = rs.standard_normal((T, n)).astype(np.float32)
    value = rs.standard_normal((T, n)).astype(np.float32)
    done = (rs.random((T, n)) < 0.2).astype(np.uint8)
    head = rs.standard_normal((n, A + 1)).astype(np.float32)
    adv, ret = orc.gae(reward, done, value, head, A, 0.99, 0.95)
    g, lam = 0.99, 0.95
    vnext = np.concatenate([value[1:], head[None, :, A]]).astype(np.float64)
    delta = reward + g * vnext * (1 - done) - value
    want = np.zeros((T, n))
    for t in range(T):
        acc, disc = np.zeros(n), np.ones(n)
        alive = np.ones(n)
        for l in range(t, T):
            acc += alive * disc * delta[l]
            alive *= 1 - done[l]
            disc *= g * lam
        want[t] = acc
    np.testing.assert_allclose(adv, want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(ret, want + value, rtol=1e-5, atol=1e-5)


# ---- minibatch order (seeded block shuffle) ------------------------------------------

def test_shuffle_is_a_seeded_permutation(orc):
    s, s2 = C.c_uint64(0), C.c_uint64(0)
    orc.lib().orc_shuffle_state_init(3, C.byref(s))
    orc.lib().orc_shuffle_state_init(3, C.byref(s2))
    a = np.arange(64, dtype=np.uint32)
    b = a.copy()
    orc.lib().orc_shuffle_blocks(C.byref(s), orc.ptr(a), 64)
    orc.lib().orc_shuffle_blocks(C.byref(s2), orc.ptr(b), 64)
    assert np.array_equal(a, b) and sorted(a) == list(range(64)) and not np.array_equal(a, np.arange(64))
    c = a.copy()
    orc.lib().orc_shuffle_blocks(C.byref(s), orc.ptr(c), 64)
    assert sorted(c) == list(range(64)) and not np.array_equal(c, a)


# ---- VoxelNav16 (navigation in a 16^3 voxel grid) -------------------------------------

def vn_fields(state):
    head = state[:32].view(np.int32)
    return head[:3].copy(), head[3:6].copy(), int(head[6]), state[32:].reshape(16, 16, 16)


def test_voxelnav_reset_and_step_spec(orc):
    rs = np.random.default_rng(9)
    occ = []
    for e in range(40):
        st = np.zeros(32 + 4096, np.uint8)
        rng = np.array([rs.integers(1, 2**32)], np.uint32)
        orc.lib().orc_env_reset(3, orc.ptr(st), orc.ptr(rng))
        pos, goal, steps, grid = vn_fields(st)
        occ.append(grid.mean())
        assert steps == 0 and not np.array_equal(pos, goal)
        assert grid[pos[2], pos[1], pos[0]] == 0 and grid[goal[2], goal[1], goal[0]] == 0
        for k in range(300):
            a = np.array([rs.integers(0, 6)], np.int32)
            before = pos.copy()
            obs, r, d = np.zeros(30, np.float32), np.zeros(1, np.float32), np.zeros(1, np.uint8)
            orc.lib().orc_env_step(3, orc.ptr(st), orc.ptr(a), orc.ptr(obs), orc.ptr(r), orc.ptr(d))
            pos, goal, steps, grid = vn_fields(st)
            delta = np.zeros(3, int)
            delta[a[0] // 2] = -1 if a[0] % 2 else 1
            target = before + delta
            inside = np.all((target >= 0) & (target < 16))
            blocked = (not inside) or grid[target[2], target[1], target[0]] == 1
            assert np.array_equal(pos, before if blocked else target)
            at_goal = np.array_equal(pos, goal)
            assert r[0] == np.float32(1.0 if at_goal else (-0.1 if blocked else -0.01))
            assert d[0] == (at_goal or steps >= 256)
            # obs: 3x3x3 neighbourhood (z, y, x order; outside = occupied) + goal delta / 15
            k2 = 0
            for dz in (-1, 0, 1):
                for dy in (-1, 0, 1):
                    for dx in (-1, 0, 1):
                        q = pos + [dx, dy, dz]
                        o = 1.0 if (np.any(q < 0) or np.any(q > 15)) else float(grid[q[2], q[1], q[0]])
                        assert obs[k2] == o
                        k2 += 1
            assert np.array_equal(obs[27:], ((goal - pos).astype(np.float32) / np.float32(15.0)))
            if d[0]:
                break
    assert abs(np.mean(occ) - 0.25) < 0.02


def test_bf16_rounding_matches_torch(orc):
    """The oracle's bfloat16 rounding against torch's float -> bfloat16 cast
    (round to nearest, ties to even), including exact ties either side."""
    import torch

    rs = np.random.default_rng(21)
    x = (rs.standard_normal(20000) * np.exp(rs.uniform(-20, 20, 20000))).astype(np.float32)
    ties = (rs.integers(1, 2**31, 2000, dtype=np.int64).astype(np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, ties.view(np.float32), np.float32([0.0, -0.0, 1.0, 65504.0, 1e-38])])
    x = x[np.isfinite(x)]  # the rounding is defined for finite values
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = np.array([orc.lib().orc_round_bf16(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", ["ppo_categorical", "ppo_voxel_shape"])
def test_bf16_forward_vs_torch(orc, name):
    """The bf16 forward: the block GEMMs' operands (LN output, up and down
    weights, relu'd hidden) rounded to bfloat16 from their fp32 values, all else
    as the fp32 forward, against a float64 torch forward with the same operand
    rounding. The fp32 forward differs from it by much more than the bound, so
    a dropped rounding point fails."""
    import torch
    import torch.nn.functional as F

    from golden import make_golden as mk

    z = load(name)
    O, A, E, H, L, cont, B = (int(x) for x in z["dims"])
    d = orc.Dims(O, A, E, H, L, cont, 1)
    head = orc.forward(d, z["params0"], z["obs"], threads=2)
    t = mk.torch_params(z["params0"], O, A, E, H, L, bool(cont))
    bf = lambda v: v.float().to(torch.bfloat16).double()
    with torch.no_grad():
        h = torch.tensor(z["obs"], dtype=torch.float64) @ t["in_w"] + t["in_b"]
        for l in range(L):
            x = F.layer_norm(h, (E,), t[f"g{l}"], t[f"b{l}"], eps=1e-5)
            v = torch.relu(bf(x) @ bf(t[f"up{l}"]))
            h = h + bf(v) @ bf(t[f"down{l}"])
        x = F.layer_norm(h, (E,), t[f"g{L}"], t[f"b{L}"], eps=1e-5)
        want = (x @ t["head"]).numpy()
    err = np.abs(head - want).max() / max(1.0, np.abs(want).max())
    fp32 = orc.forward(orc.Dims(O, A, E, H, L, cont, 0), z["params0"], z["obs"], threads=2)
    gap = np.abs(fp32 - want).max() / max(1.0, np.abs(want).max())
    assert err < 2e-4, err
    assert gap > 10 * err, (gap, err)


@pytest.mark.parametrize("name", ["ppo_categorical", "ppo_gaussian"])
def test_bf16_ppo_gradient_vs_torch(orc, name):
    """The bf16 train step's gradient against torch autograd through a matmul
    that rounds its operands to bfloat16 (from their fp32 values) in the
    forward and rounds the incoming gradient and the saved operands in the
    backward: with the block matmuls built from it, autograd places every
    rounding point the bf16 mode defines (dV = q(dh) q(Down)^T, dx = q(dV)
    q(Up)^T, dUp = q(x)^T q(dV), dDown = q(V)^T q(dh)), independently of the
    oracle's loops. Flipped roundings bound the agreement (measured 1e-4 and
    below per parameter group); the fp32 gradient is 10-100x further away."""
    import torch
    import torch.nn.functional as F

    from golden import make_golden as mk

    def q(v):
        return v.float().to(torch.bfloat16).double()

    class BfMatmul(torch.autograd.Function):
        @staticmethod
        def forward(ctx, a, w):
            ctx.save_for_backward(a, w)
            return q(a) @ q(w)

        @staticmethod
        def backward(ctx, g):
            a, w = ctx.saved_tensors
            return q(g) @ q(w).T, q(a).T @ q(g)

    z = load(name)
    O, A, E, H, L, cont, B = (int(x) for x in z["dims"])
    clip, vc, ec, mgn, gamma, lam, lr = z["hp"]
    hp = orc.hparams(clip=clip, value_coef=vc, entropy_coef=ec, max_grad_norm=mgn, lr=lr)
    grads = {}
    for bf in (1, 0):
        d = orc.Dims(O, A, E, H, L, cont, bf)
        P, M, V = z["params0"].copy(), np.zeros_like(z["params0"]), np.zeros_like(z["params0"])
        _, grads[bf], _ = orc.train_minibatch(d, hp, P, M, V, 1, z["obs"], z["actions"], z["adv"], z["ret"],
                                               z["old_logp"], threads=2)
    t = mk.torch_params(z["params0"], O, A, E, H, L, bool(cont))
    h = torch.tensor(z["obs"], dtype=torch.float64) @ t["in_w"] + t["in_b"]
    for l in range(L):
        x = F.layer_norm(h, (E,), t[f"g{l}"], t[f"b{l}"], eps=1e-5)
        h = h + BfMatmul.apply(torch.relu(BfMatmul.apply(x, t[f"up{l}"])), t[f"down{l}"])
    x = F.layer_norm(h, (E,), t[f"g{L}"], t[f"b{L}"], eps=1e-5)
    head = x @ t["head"]
    act = torch.tensor(z["actions"], dtype=torch.float64 if cont else torch.int64)
    f64 = lambda a: torch.tensor(a, dtype=torch.float64)
    loss, _, _ = mk.ppo_loss(head, A, bool(cont), t, act, f64(z["adv"]), f64(z["ret"]), f64(z["old_logp"]), clip,
                             vc, ec)
    loss.backward()
    off, count = mk.layout(O, A, E, H, L, bool(cont))
    want = np.zeros(count)
    for k, v in t.items():
        want[off[k]:off[k] + v.numel()] = v.grad.numpy().ravel()
    for k in ("up0", "down0", f"up{L - 1}", f"down{L - 1}", "in_w", "head", "g0", "b0"):
        o, c = off[k], t[k].numel()
        w = want[o:o + c]
        e_bf = np.linalg.norm(grads[1][o:o + c] - w) / np.linalg.norm(w)
        e_fp = np.linalg.norm(grads[0][o:o + c] - w) / np.linalg.norm(w)
        print(f"{k}: bf16 oracle vs torch {e_bf:.2e}, fp32 oracle vs torch {e_fp:.2e}")
        assert e_bf < 1e-3, (k, e_bf)
        assert e_fp > 10 * e_bf, (k, e_fp, e_bf)


@pytest.mark.parametrize("name", ["ppo_categorical", "ppo_gaussian"])
def test_masked_train_step_vs_torch(orc, name):
    """The oracle's ReLU-mask override (the GPU gradient gate replays the GPU's
    ReLU decisions through it) against torch float64 autograd of the function
    the mask defines: each block's hidden units are its pre-activations times
    a fixed 0/1 mask. The mask is the oracle's own z > 0 with a few hundred
    decisions inverted, including units far from 0, so a mask applied only in
    the forward or only in the backward, or ignored, fails. With the mask equal
    to z > 0 the step is bit for bit the unmasked one."""
    import torch
    import torch.nn.functional as F

    from golden import make_golden as mk

    z = load(name)
    O, A, E, H, L, cont, B = (int(x) for x in z["dims"])
    d = orc.Dims(O, A, E, H, L, cont, 0)
    clip, vc, ec, mgn, gamma, lam, lr = z["hp"]
    hp = orc.hparams(clip=clip, value_coef=vc, entropy_coef=ec, max_grad_norm=mgn, lr=lr)
    args = (z["obs"], z["actions"], z["adv"], z["ret"], z["old_logp"])
    fresh = lambda: (z["params0"].copy(), np.zeros_like(z["params0"]), np.zeros_like(z["params0"]))
    P0, M0, V0 = fresh()
    _, g_plain, _ = orc.train_minibatch(d, hp, P0, M0, V0, 1, *args, threads=2)
    P1, M1, V1 = fresh()
    _, g_own, _, pre = orc.train_minibatch_masked(d, hp, P1, M1, V1, 1, *args, None, threads=2)
    P2, M2, V2 = fresh()
    _, g_same, _, _ = orc.train_minibatch_masked(d, hp, P2, M2, V2, 1, *args, pre > 0, threads=2)
    assert np.array_equal(g_plain, g_own) and np.array_equal(g_plain, g_same)
    assert np.array_equal(P0, P2) and np.array_equal(M0, M2) and np.array_equal(V0, V2)
    rs = np.random.default_rng(11)
    mask = pre > 0
    flip = rs.random(mask.shape) < 0.05
    mask ^= flip
    P3, M3, V3 = fresh()
    _, g_mask, _, pre3 = orc.train_minibatch_masked(d, hp, P3, M3, V3, 1, *args, mask, threads=2)
    # torch: the same network with relu(z) replaced by z * mask
    t = mk.torch_params(z["params0"], O, A, E, H, L, bool(cont))
    mt = torch.tensor(mask, dtype=torch.float64)
    h = torch.tensor(z["obs"], dtype=torch.float64) @ t["in_w"] + t["in_b"]
    zs = []
    for l in range(L):
        x = F.layer_norm(h, (E,), t[f"g{l}"], t[f"b{l}"], eps=1e-5)
        zl = x @ t[f"up{l}"]
        zs.append(zl.detach().numpy())
        h = h + (zl * mt[:, l, :]) @ t[f"down{l}"]
    x = F.layer_norm(h, (E,), t[f"g{L}"], t[f"b{L}"], eps=1e-5)
    head = x @ t["head"]
    act = torch.tensor(z["actions"], dtype=torch.float64 if cont else torch.int64)
    f64 = lambda a: torch.tensor(a, dtype=torch.float64)
    loss, _, _ = mk.ppo_loss(head, A, bool(cont), t, act, f64(z["adv"]), f64(z["ret"]), f64(z["old_logp"]), clip, vc,
                             ec)
    loss.backward()
    off, count = mk.layout(O, A, E, H, L, bool(cont))
    want = np.zeros(count)
    for k, v in t.items():
        want[off[k]:off[k] + v.numel()] = v.grad.numpy().ravel()
    np.testing.assert_allclose(pre3, np.stack(zs, axis=1), rtol=1e-4, atol=1e-5)
    assert rel_group_err(g_mask, want) < 2e-5
    assert rel_group_err(g_plain, want) > 100 * rel_group_err(g_mask, want)
