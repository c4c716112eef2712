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
