"""Shared helpers of the GPU parity tests: the tolerances of each compared quantity."""
import os

import numpy as np

THREADS = min(16, os.cpu_count() or 1)

ENVS = {
    "cartpole": (0, "rollout_cartpole"),
    "cartpole_continuous": (1, "rollout_cartpole_continuous"),
    "cartpole_continuous_clamp": (2, "rollout_cartpole_continuous_clamp"),
    "voxelnav16": (3, "rollout_voxelnav16"),
    "voxelnav": (4, "rollout_voxelnav"),
}

TOL_HEAD = 1e-4     # policy head, values, GAE
TOL_TRAIN = 1e-3    # LossStats, post-Adam weights


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def assert_bit_exact(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    bad = np.flatnonzero(bits(got).ravel() != bits(want).ravel())
    assert bad.size == 0, f"{what}: {bad.size} of {got.size} differ; first at {bad[:5]}: {got.ravel()[bad[:5]]} vs {want.ravel()[bad[:5]]}"


def assert_close(got, want, tol, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    worst = float(err.max()) if err.size else 0.0
    assert worst <= tol, f"{what}: max scaled error {worst:.3g} > {tol} at {np.unravel_index(err.argmax(), err.shape)}"
    return worst


# bf16 mode: operands are rounded to bfloat16 from fp32 values whose last bits
# depend on the summation order, so where an operand sits on a rounding
# boundary the two sides round it one bf16 ulp (2^-8) apart and that row's
# outputs move by up to ~1e-3 per flip. Measured on the CPU (the oracle against
# numpy-ordered GEMMs with the same rounding points): median 0, 0.6% of rows
# above 1e-5, 99.9th percentile 2e-4, worst 1e-3; the GPU's summation order
# differs more, so more rows flip. A wrong or missing rounding point moves
# every row by ~1e-3 (bf16 against fp32: 9e-3), which the median catches.
TOL_BF16_MEDIAN = 1e-5
TOL_BF16_P99 = 3e-3
TOL_BF16_MAX = 2e-2


def assert_close_bf16(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = (np.abs(got - want) / np.maximum(1.0, np.abs(want))).ravel()
    if err.size == 0:
        return 0.0
    med, p99, worst = float(np.median(err)), float(np.quantile(err, 0.99)), float(err.max())
    print(f"{what}: median {med:.2e} p90 {np.quantile(err, 0.9):.2e} p99 {p99:.2e} max {worst:.2e} "
          f"above 1e-5: {(err > 1e-5).mean():.3f}")
    assert med <= TOL_BF16_MEDIAN, f"{what}: median scaled error {med:.3g} > {TOL_BF16_MEDIAN}"
    assert p99 <= TOL_BF16_P99, f"{what}: 99th percentile scaled error {p99:.3g} > {TOL_BF16_P99}"
    assert worst <= TOL_BF16_MAX, f"{what}: max scaled error {worst:.3g} > {TOL_BF16_MAX}"
    return worst


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


TOL_MOMENT = 1e-3   # Adam moments per parameter group, relative L2, against the mask-matched oracle
TOL_FLIP = 1e-5     # |z| of a flipped ReLU unit relative to ||x_row|| ||Up[:, j]||


def check_minibatch(model, orc, d, hp, p0, rows, B, step=1):
    """One fp32 minibatch update of the GPU against the oracle evaluating the
    same function: the oracle replays the GPU's ReLU decisions (read from the
    row pass's hidden capture), so a pre-activation that two summation orders
    put on either side of 0 counts as the same unit. Then, with no exemptions:
    - the recomputed head within TOL_HEAD;
    - both Adam moments of every parameter group within TOL_MOMENT relative L2
      (after one step from zero moments they are 0.1 g and 0.001 g^2 of the
      clipped gradient, so this holds the gradient itself);
    - every flipped unit's pre-activation is within rounding of 0: |z| <=
      TOL_FLIP ||x_row|| ||Up[:, j]||, z as the oracle computes it;
    - LossStats within TOL_TRAIN (clip_frac within two rows) and the post-Adam
      weights within TOL_TRAIN.
    Returns the oracle's (stats, params) after the step."""
    pv = model.pv
    m1, v1, st_gpu = model.adam_state()
    assert st_gpu == step
    hid = model.train_capture(1)  # [L][B][H]
    x = model.train_capture(0)    # [L][B][E]
    mask = np.ascontiguousarray((hid > 0).transpose(1, 0, 2))
    P, M, V = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    st, grad, head, pre = orc.train_minibatch_masked(d, hp, P, M, V, step, *rows, mask, threads=THREADS)
    assert_close(model.head(), head, TOL_HEAD, "recomputed head")
    em, ev = group_errors(pv, m1, M), group_errors(pv, v1, V)
    flips = (pre > 0) != mask
    nflip = int(flips.sum())
    worst = 0.0
    if nflip:
        r, l, j = np.nonzero(flips)
        E, H = pv.embed, pv.hidden
        upn = np.stack([np.linalg.norm(p0[pv.off_up[k]:pv.off_up[k] + E * H].reshape(E, H).astype(np.float64), axis=0)
                        for k in range(pv.layers)])
        scale = np.linalg.norm(x.transpose(1, 0, 2)[r, l].astype(np.float64), axis=-1) * upn[l, j]
        rel = np.abs(pre[r, l, j]) / scale
        worst = float(rel.max())
    print(f"ReLU units on the other side of 0: {nflip} of {mask.size} (worst |z| / scale {worst:.2e}); "
          f"moment m worst {max(em.values()):.2e} ({max(em, key=em.get)}), v worst {max(ev.values()):.2e}")
    assert worst <= TOL_FLIP, f"a flipped ReLU unit's pre-activation is {worst:.3g} of its scale"
    bad = {k: e for k, e in em.items() if e >= TOL_MOMENT}
    assert not bad, f"first moment (gradient) differs: {bad}"
    bad = {k: e for k, e in ev.items() if e >= TOL_MOMENT}
    assert not bad, f"second moment differs: {bad}"
    got, want = np.array(model.last_stats().as_tuple()), np.array(st.as_tuple())
    assert_close(got[[0, 1, 2, 3, 5]], want[[0, 1, 2, 3, 5]], TOL_TRAIN, "LossStats")
    assert abs(got[4] - want[4]) * B <= 2.0 + 1e-3, (got[4], want[4])
    p1 = model.params()
    assert_close(p1, P, TOL_TRAIN, "post-Adam weights")
    assert np.all(np.isfinite(p1))
    return st, P
