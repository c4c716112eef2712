"""Shared helpers of the GPU parity tests (tolerances from BASELINE.json's north_star)."""
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
