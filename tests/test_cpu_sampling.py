"""Pins the oracle's samplers and its collect sequencing, independently of the
oracle's own loops:

- the categorical draw (model/sample.metal:18-47) against the inverse-CDF
  closed form in float64, with draws placed exactly on a CDF boundary (the
  `u < cumsum` comparison decides them) and exactly one RNG draw per row;
- the Gaussian draw (model/gaussian.metal:32-38, 59-69) against Box-Muller in
  float64 from the same two uniforms (u1 = 1 - u, cos for even, sin for odd
  action dimensions, two draws per pair);
- collect (model/ppo.h:716-751, rollout.h:46-47) against a replay built from
  separately pinned pieces: the extra first step with action 0, then per step
  forward -> sample -> reset-if-done -> step, the obs[T] -> obs[0] copy on the
  next call, the bootstrap forward; and against an RNG draw count.
"""
import ctypes as C
import math

import numpy as np
import pytest

M32 = 0xFFFFFFFF


def xorshift(s):
    """Marsaglia xorshift32, shifts 13/17/5 (rollout.h:9-14)."""
    s ^= (s << 13) & M32
    s ^= s >> 17
    s ^= (s << 5) & M32
    return s & M32


def xorshift_inverse(y):
    """The state whose next xorshift32 output is y."""
    x = y
    for _ in range(7):  # undo s ^= s << 5 (fixed point after ceil(32 / 5) rounds)
        x = (y ^ (x << 5)) & M32
    x ^= x >> 17        # undo s ^= s >> 17
    y2 = x
    x = (y2 ^ (y2 << 13) ^ (y2 << 26)) & M32  # undo s ^= s << 13
    return x


def test_xorshift_inverse_roundtrip():
    rs = np.random.default_rng(3)
    for s in rs.integers(1, 2**32, 500):
        s = int(s)
        assert xorshift_inverse(xorshift(s)) == s and xorshift(xorshift_inverse(s)) == s


def state_for_uniform_k(k, low=0x5A):
    """An RNG state whose next draw gives (x >> 8) == k."""
    assert 0 <= k < 2**24
    return xorshift_inverse((k << 8) | low)


def sample(orc, d, params, head, rng):
    rows = head.shape[0]
    head = np.ascontiguousarray(head, np.float32)
    rng = np.ascontiguousarray(rng, np.uint32).copy()
    acts = np.zeros((rows, d.act_dim) if d.continuous else (rows,), np.float32 if d.continuous else np.int32)
    logp = np.zeros(rows, np.float32)
    value = np.zeros(rows, np.float32)
    orc.lib().orc_sample(C.byref(d), orc.ptr(params), orc.ptr(head), rows, orc.ptr(rng), orc.ptr(acts),
                         orc.ptr(logp), orc.ptr(value))
    return acts, logp, value, rng


def params_for(orc, d):
    return orc.init_params(d, 0)


# ---- categorical (model/sample.metal:18-47) -------------------------------------------


def categorical_f64(h, k):
    """Inverse CDF in float64: u = k 2^-24 sum exp(z - max); the first a with
    u < cumsum_a, default A - 1. Returns (action, log-softmax row, u, cdf)."""
    z = np.asarray(h, np.float64)
    e = np.exp(z - z.max())
    cdf = np.cumsum(e)
    u = k * 2.0**-24 * cdf[-1]
    hit = np.flatnonzero(u < cdf)
    a = int(hit[0]) if hit.size else len(z) - 1
    return a, z - z.max() - math.log(cdf[-1]), u, cdf


@pytest.mark.parametrize("A", [2, 6, 63])
def test_categorical_matches_inverse_cdf(orc, A):
    """Random heads (wide and near-tied logits) and random RNG states against the
    float64 closed form; rows whose u is within float rounding of a CDF boundary
    may land on either neighbour, all others must match exactly."""
    d = orc.Dims(4, A, 128, 512, 2, 0, 0)
    P = params_for(orc, d)
    rs = np.random.default_rng(100 + A)
    rows = 4000
    head = np.zeros((rows, A + 1), np.float32)
    head[: rows // 2, :A] = rs.standard_normal((rows // 2, A)) * 3.0
    base = rs.standard_normal((rows - rows // 2, 1))
    head[rows // 2:, :A] = base + rs.standard_normal((rows - rows // 2, A)) * 1e-6  # near ties
    head[:, A] = rs.standard_normal(rows)
    rng0 = rs.integers(1, 2**32, rows, dtype=np.uint64).astype(np.uint32)
    acts, logp, value, rng1 = sample(orc, d, P, head, rng0)
    decided = 0
    for r in range(rows):
        nxt = xorshift(int(rng0[r]))
        assert rng1[r] == nxt, "exactly one draw per row"
        a, lsm, u, cdf = categorical_f64(head[r, :A], nxt >> 8)
        near = np.abs(u - cdf) <= 1e-5 * cdf[-1]
        if not near.any():
            decided += 1
            assert acts[r] == a, (r, acts[r], a)
        else:
            lo = int(np.flatnonzero(near)[0])
            assert acts[r] in (a, lo, lo + 1), (r, acts[r], a)
        assert abs(logp[r] - lsm[acts[r]]) <= 2e-6 * max(1.0, abs(lsm[acts[r]])), (r, logp[r], lsm[acts[r]])
        assert value[r] == head[r, A]
    assert decided > 0.9 * rows


def zeros_logits(A):
    return np.zeros(A, np.float32) + np.float32(0.75)  # equal logits: exp(z - max) = exp(0) = 1 exactly


def half_masked_logits(A):
    """Logit 0 at even indices, -100 at odd ones: exp(-100) is exactly 0 on the
    float path, so the CDF is 1, 1, 2, 2, ... and the sum is a power of two."""
    z = np.full(A, -100.0, np.float32)
    z[0::2] = 0.0
    return z


@pytest.mark.parametrize("logits,k,want", [
    (zeros_logits(2), 2**23, 1),          # u = 1.0 exactly = cdf[0]: u < cdf[0] fails, action 1
    (zeros_logits(2), 2**23 - 1, 0),      # just below the boundary
    (zeros_logits(4), 2**22, 1),          # u = 1.0 = cdf[0]
    (zeros_logits(4), 3 * 2**22, 3),      # u = 3.0 = cdf[2]
    (zeros_logits(6), 2**23, 3),          # u = 3.0 = cdf[2]
    (zeros_logits(6), 2**24 - 1, 5),      # the top draw: the last action
    (zeros_logits(6), 0, 0),              # u = 0 < cdf[0]
    (half_masked_logits(63), 5 * 2**19, 10),  # u = 5 = cdf[8] = cdf[9]; cdf[10] = 6
    (half_masked_logits(63), 5 * 2**19 - 1, 8),
])
def test_categorical_exact_cdf_boundaries(orc, logits, k, want):
    """With exp values of exactly 1 (or 0) the CDF holds small integers and
    u = k 2^-24 sum is exact: a draw exactly on a boundary goes to the next
    action with non-zero probability (the comparison is u < cumsum, not <=)."""
    A = logits.size
    assert orc.lib().orc_expf(-100.0) == 0.0
    d = orc.Dims(4, A, 128, 512, 2, 0, 0)
    P = params_for(orc, d)
    head = np.zeros((1, A + 1), np.float32)
    head[0, :A] = logits
    rng0 = np.array([state_for_uniform_k(k)], np.uint32)
    acts, logp, _, rng1 = sample(orc, d, P, head, rng0)
    assert acts[0] == want
    assert rng1[0] == xorshift(int(rng0[0]))
    z = logits.astype(np.float64)
    lsm = z - z.max() - math.log(np.exp(z - z.max()).sum())
    assert abs(logp[0] - lsm[want]) <= 1e-6


def test_categorical_boundary_with_unequal_logits(orc):
    """cdf = (1, 3) from logits (0, ln 2) is not exact in float (exp(ln 2 - ln 2)
    = 1 for the max, exp(-ln 2) ~ 0.5): place u just either side of cdf[0] by
    k, with a margin of a few float ulps, to pin which side is which."""
    d = orc.Dims(4, 2, 128, 512, 2, 0, 0)
    P = params_for(orc, d)
    head = np.array([[0.0, math.log(2.0), 0.0]], np.float32)
    e0 = math.exp(float(head[0, 0]) - float(head[0, 1]))
    S = e0 + 1.0
    kb = e0 / S * 2**24  # boundary in k units
    for k, want in ((int(kb) - 64, 0), (int(kb) + 64, 1)):
        rng0 = np.array([state_for_uniform_k(k)], np.uint32)
        acts, _, _, _ = sample(orc, d, P, head, rng0)
        assert acts[0] == want, (k, kb, acts[0])


# ---- Gaussian (model/gaussian.metal:32-38, 59-69) ---------------------------------------


def gaussian_f64(mu, ls, s):
    """Box-Muller from the draws after state s: per pair, u1 = 1 - k1 2^-24,
    u2 = k2 2^-24, r = sqrt(-2 ln u1), z = r cos(2 pi u2) for the even and
    r sin(2 pi u2) for the odd dimension. Returns (action, logp, state)."""
    A = len(mu)
    a = np.zeros(A)
    z = (0.0, 0.0)
    for k in range(A):
        if k % 2 == 0:
            s = xorshift(s)
            u1 = 1.0 - (s >> 8) * 2.0**-24
            s = xorshift(s)
            u2 = (s >> 8) * 2.0**-24
            r = math.sqrt(-2.0 * math.log(u1))
            z = (r * math.cos(2 * math.pi * u2), r * math.sin(2 * math.pi * u2))
        a[k] = mu[k] + math.exp(ls[k]) * z[k % 2]
    dd = (a - mu) * np.exp(-np.asarray(ls, np.float64))
    logp = float(np.sum(-0.5 * dd * dd - np.asarray(ls) - 0.5 * math.log(2 * math.pi)))
    return a, logp, s


@pytest.mark.parametrize("A", [1, 2, 3])
def test_gaussian_matches_box_muller(orc, A):
    d = orc.Dims(4, A, 128, 512, 2, 1, 0)
    P = params_for(orc, d).copy()
    L = orc.layout(d)
    ls = np.array([-0.7, 0.4, 0.15][:A], np.float32)
    P[L.off_log_std:L.off_log_std + A] = ls
    rs = np.random.default_rng(200 + A)
    rows = 3000
    head = rs.standard_normal((rows, A + 1)).astype(np.float32)
    rng0 = rs.integers(1, 2**32, rows, dtype=np.uint64).astype(np.uint32)
    # the extreme draws: u1 = 1 (r = 0) and u1 = 2^-24 (the largest radius)
    rng0[0] = state_for_uniform_k(0)
    rng0[1] = state_for_uniform_k(2**24 - 1)
    acts, logp, value, rng1 = sample(orc, d, P, head, rng0)
    acts = acts.reshape(rows, A)
    for r in range(rows):
        a, lp, s = gaussian_f64(head[r, :A].astype(np.float64), ls.astype(np.float64), int(rng0[r]))
        assert rng1[r] == s, "two draws per pair of action dimensions"
        np.testing.assert_allclose(acts[r], a, rtol=0, atol=3e-6 * (1 + np.abs(a).max()))
        assert abs(logp[r] - lp) <= 2e-5 * max(1.0, abs(lp)), (r, logp[r], lp)
        assert value[r] == head[r, A]
    assert np.all(acts[0, :2] == head[0, :min(A, 2)])  # u1 = 1 in the first pair: r = 0


# ---- collect sequencing (model/ppo.h:716-751) -----------------------------------------


def env_ptrs(g, i):
    sb = g.info.state_bytes
    return g.state.ctypes.data + i * sb, g.rng.ctypes.data + 4 * i


def env_step_one(orc, g, i, act, O):
    """rollout.h:46-52 for env i: reset if done, then step (obs and reward start
    at zero)."""
    sp, rp = env_ptrs(g, i)
    if g.done[i]:
        orc.lib().orc_env_reset(g.env, C.c_void_p(sp), C.c_void_p(rp))
    obs = np.zeros(O, np.float32)
    r = np.zeros(1, np.float32)
    dn = np.zeros(1, np.uint8)
    a = np.ascontiguousarray(act)
    orc.lib().orc_env_step(g.env, C.c_void_p(sp), orc.ptr(a), orc.ptr(obs), orc.ptr(r), orc.ptr(dn))
    g.done[i] = dn[0]
    return obs, r[0]


def replay_collect(orc, g, d, params, T, first, prev_obs_T=None):
    """model/ppo.h:716-751 restated from the pinned pieces: forward (torch
    fixtures), sampling (closed forms above), env reset/step (textbook
    equations), called in the reference's order."""
    n, O, A = g.n, d.obs_dim, d.act_dim
    cont = bool(d.continuous)
    obs = np.zeros((T + 1, n, O), np.float32)
    acts = np.zeros((T, n, A) if cont else (T, n), np.float32 if cont else np.int32)
    logp = np.zeros((T, n), np.float32)
    value = np.zeros((T, n), np.float32)
    reward = np.zeros((T, n), np.float32)
    done = np.zeros((T, n), np.uint8)
    if first:  # model/ppo.h:720-722: one step with the zeroed action slot 0
        zero = np.zeros(A, np.float32) if cont else np.zeros(1, np.int32)
        for i in range(n):
            obs[0, i], reward[0, i] = env_step_one(orc, g, i, zero, O)
    else:  # model/ppo.h:724: obs slot T of the previous rollout becomes slot 0
        obs[0] = prev_obs_T
    for t in range(T):
        head = orc.forward(d, params, obs[t], threads=2)  # :728
        a, lp, v, rng = sample(orc, d, params, head, g.rng)  # :729 (draws before the step's reset)
        g.rng[:] = rng
        acts[t], logp[t], value[t] = a.reshape(acts[t].shape), lp, v
        for i in range(n):  # :730, rollout.h:46-52
            obs[t + 1, i], reward[t, i] = env_step_one(orc, g, i, acts[t, i], O)
        done[t] = g.done  # :732
    head = orc.forward(d, params, obs[T], threads=2)  # :735 bootstrap
    return dict(obs=obs, actions=acts, logp=logp, value=value, reward=reward, done=done, head=head)


def draws_per_sample(d):
    return 2 * ((d.act_dim + 1) // 2) if d.continuous else 1


@pytest.mark.parametrize("env", [0, 1, 3])
def test_collect_matches_reference_order(orc, env):
    """Two consecutive collects (the first with its extra action-0 step, the
    second starting from the copied obs[T]) bit for bit against the replay:
    obs, actions, log-probs, values, rewards, dones, RNG, env state and the
    bootstrap head; GAE on the replay's slots."""
    n, T = 48, 16 if env != 3 else 6
    d = orc.dims(env)
    params = orc.init_params(d, 0)
    if d.continuous:
        params = params.copy()
        params[orc.layout(d).off_log_std] = -0.3  # exercise exp(log_std)
    g = orc.GymState(env, n, 0)
    g_rep = g.copy()
    prev = None
    saw_done = False
    slots = orc.Slots(env, n, T)  # persistent, as the model's slots: call 2 reads its obs[T]
    for call in range(2):
        orc.collect(g, d, params, T, slots, first=(call == 0), threads=2)
        want = replay_collect(orc, g_rep, d, params, T, call == 0, prev)
        for key, got in (("obs", slots.obs), ("actions", slots.actions), ("logp", slots.logp),
                         ("value", slots.value), ("reward", slots.reward), ("done", slots.done), ("head", slots.head)):
            np.testing.assert_array_equal(np.ascontiguousarray(got).view(np.uint8),
                                          np.ascontiguousarray(want[key]).view(np.uint8), err_msg=f"call {call} {key}")
        np.testing.assert_array_equal(slots.value, slots_value_from_head(orc, d, params, slots.obs[:T]))
        assert np.array_equal(g.rng, g_rep.rng) and np.array_equal(g.state, g_rep.state)
        assert np.array_equal(g.done, g_rep.done)
        adv, ret = orc.gae(want["reward"], want["done"], want["value"], want["head"], d.act_dim)
        np.testing.assert_array_equal(slots.adv, adv)
        np.testing.assert_array_equal(slots.ret, ret)
        prev = slots.obs[T].copy()
        saw_done |= bool(slots.done[:-1].any())
    assert saw_done or env == 3  # episodes ended inside the rollouts, so resets ran between sample and step


def slots_value_from_head(orc, d, params, obs_slots):
    """The value slot is column ACT_DIM of the forward of the same obs slot."""
    T, n, O = obs_slots.shape
    head = orc.forward(d, params, obs_slots.reshape(T * n, O), threads=2)
    return head[:, d.act_dim].reshape(T, n)


@pytest.mark.parametrize("env", [0, 1])
def test_collect_rng_accounting(orc, env):
    """CartPole resets take 4 draws. First call: 4 per env for the extra
    action-0 step (done starts at 1) and no sampling draw; then per step the
    sampler's draws (1 categorical, 2 per pair of Gaussian dimensions) plus 4
    when the previous step ended the episode. The second call adds no extra
    step."""
    n, T = 256, 40
    d = orc.dims(env)
    params = orc.init_params(d, 0)
    g = orc.GymState(env, n, 0)
    rng0 = g.rng.copy()
    slots = orc.Slots(env, n, T)
    orc.collect(g, d, params, T, slots, first=True, threads=4)
    per = draws_per_sample(d)
    # done after the extra step is invisible in the slots, so count it by replaying
    # the extra step alone on a copy
    g1 = orc.GymState(env, n, 0)
    zero = np.zeros(d.act_dim, np.float32) if d.continuous else np.zeros(1, np.int32)
    for i in range(n):
        env_step_one(orc, g1, i, zero, d.obs_dim)
    done_before = np.concatenate([g1.done[None], slots.done[:-1]]).astype(int)
    counts = 4 + T * per + 4 * done_before.sum(axis=0)
    for i in range(n):
        s = int(rng0[i])
        for _ in range(counts[i]):
            s = xorshift(s)
        assert s == g.rng[i], i
    assert done_before.sum() > 0
    rng1 = g.rng.copy()
    last_done = slots.done[-1].astype(int)
    obs_T = slots.obs[T].copy()
    slots2 = slots
    orc.collect(g, d, params, T, slots2, first=False, threads=4)
    np.testing.assert_array_equal(slots2.obs[0], obs_T)
    done_before2 = np.concatenate([last_done[None], slots2.done[:-1]]).astype(int)
    counts2 = T * per + 4 * done_before2.sum(axis=0)
    for i in range(n):
        s = int(rng1[i])
        for _ in range(counts2[i]):
            s = xorshift(s)
        assert s == g.rng[i], i
