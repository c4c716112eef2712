"""collect() and one PPO minibatch at the largest policy shape the library
accepts: 64 observation floats and a 64-column head (63 logits or Gaussian
means plus the value), through two test-only envs built as a separate env
library (tests/envs, registered with MG_DEFINE_ENV like a user's env). The
oracle has no model of these envs' dynamics, so collect is checked on its
policy side: the values, log-probabilities and bootstrap head the GPU wrote
against the oracle's forward of the GPU's own observation slots (1e-4); the
minibatch against the oracle's train step on the GPU's rollout, with the
GPU's ReLU decisions replayed (head 1e-4, Adam moments, post-Adam weights and
LossStats 1e-3)."""
import ctypes
import os

import numpy as np
import pytest

from parity import THREADS, TOL_HEAD, assert_bit_exact, assert_close, check_minibatch
from test_gpu_train import block_rows

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "envs", "build", "libmg_test_envs.so")
KERNELS = {False: "rollout_test_wide64", True: "rollout_test_wide64_gauss"}


@pytest.fixture(scope="module")
def wide(mg):
    assert os.path.exists(LIB), f"{LIB} missing: run __graft_entry__.build()"
    ctypes.CDLL(LIB)  # its static initialisers register both envs with the loaded library
    assert set(KERNELS.values()) <= set(mg.env_names())
    return mg


def policy_logp(head, actions, A, cont, log_std):
    """log-probability of the taken actions under the head, in float64."""
    h = head.astype(np.float64)
    if cont:
        ls = log_std.astype(np.float64)
        d = (actions.astype(np.float64) - h[..., :A]) * np.exp(-ls)
        return (-0.5 * d * d - ls - 0.5 * np.log(2 * np.pi)).sum(-1)
    z = h[..., :A]
    lse = z.max(-1) + np.log(np.exp(z - z.max(-1, keepdims=True)).sum(-1))
    return np.take_along_axis(z, actions[..., None].astype(np.int64), -1)[..., 0] - lse


@pytest.mark.parametrize("cont", [False, True])
@pytest.mark.parametrize("n,T", [(2048, 3), (8192, 2), (32768, 2)])  # 16-, 32- and 64-row tiles
def test_wide_collect_policy_side(wide, orc, cont, n, T):
    mg = wide
    gym = mg.Gym(KERNELS[cont], n, 0)
    model = mg.PPOModel(gym, horizon=T)
    d = orc.Dims(64, 63, 128, 512, 2, int(cont))
    params = orc.init_params(d, 0)
    assert_bit_exact(model.params(), params, "initial parameters")
    pv = model.pv
    log_std = params[pv.off_log_std:pv.off_log_std + 63] if cont else None
    for c in range(2):
        model.collect()
        s = model.download_slots()
        heads = orc.forward(d, params, s["obs"][:T].reshape(T * n, 64), threads=THREADS).reshape(T, n, 64)
        assert_close(s["value"], heads[..., 63], TOL_HEAD, f"collect {c} values")
        lp = policy_logp(heads, s["actions"], 63, cont, log_std)
        assert_close(s["logp"], lp.astype(np.float32), TOL_HEAD, f"collect {c} logp")
        boot = orc.forward(d, params, s["obs"][T], threads=THREADS)
        assert_close(model.head(), boot, TOL_HEAD, f"collect {c} bootstrap head")
        assert np.isfinite(s["reward"]).all()


@pytest.mark.parametrize("cont", [False, True])
def test_wide_minibatch(wide, orc, cont):
    mg = wide
    n, T, B, block = 1024, 2, 512, 1
    gym = mg.Gym(KERNELS[cont], n, 3)
    model = mg.PPOModel(gym, horizon=T, seed=3, minibatch=B)
    d = orc.Dims(64, 63, 128, 512, 2, int(cont))
    model.collect()
    s = model.download_slots()
    p0 = model.params()
    hp = orc.hparams()
    model.train_block(block)
    check_minibatch(model, orc, d, hp, p0, block_rows(s, n, B, block), B)
