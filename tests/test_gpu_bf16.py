"""The bf16 precision mode (the reference's matmul precision: bfloat16
operands, fp32 accumulation) against the oracle's bf16 forward, which rounds
the same operands (LN output, weights, relu'd hidden) from their fp32 values.
Both sides then differ only in fp32 summation order, plus a rare 1-ulp bf16
flip where an operand's fp32 value sits on a rounding boundary; the policy
side is held to fp32 agreement at the median with flipped rows bounded
(parity.assert_close_bf16). The env side stays bit-exact under teacher
forcing."""
import numpy as np
import pytest

from parity import ENVS, THREADS, assert_close_bf16
from test_gpu_collect import run_collect_parity

pytestmark = pytest.mark.gpu

@pytest.mark.parametrize("env,n,T", [
    ("cartpole", 1024, 8),           # 16-row tiles, 8 waves
    ("cartpole", 8192, 4),           # 32-row tiles
    ("cartpole", 64 * 576, 2),       # 64-row tiles
    ("cartpole_continuous", 2048, 4),
    ("voxelnav16", 1024, 4),         # 16-row tiles, 4 waves
    ("voxelnav", 1024, 4),           # heightmaps staged in LDS beside the bf16 tiles
    ("voxelnav", 16384, 2),          # 32-row tiles, heightmaps in device memory
    ("voxelnav", 32768, 2),          # 64-row tiles, the same
])
def test_bf16_collect_teacher_forced(mg, orc, env, n, T):
    run_collect_parity(mg, orc, env, n, T, bf16=True)


@pytest.mark.parametrize("env", ["cartpole", "voxelnav"])
def test_bf16_forward_matches_oracle_and_differs_from_fp32(mg, orc, env):
    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, 256, 0)
    model = mg.PPOModel(gym, horizon=4, precision="bf16")
    rs = np.random.default_rng(5)
    obs = (rs.standard_normal((1000, gym.obs_dim)) * 3).astype(np.float32)
    head = model.forward(obs)
    want = orc.forward(orc.dims(eid, bf16=True), model.params(), obs, threads=THREADS)
    err = assert_close_bf16(head, want, "bf16 head")
    fp32 = orc.forward(orc.dims(eid), model.params(), obs, threads=THREADS)
    gap = float((np.abs(head - fp32) / np.maximum(1.0, np.abs(fp32))).max())
    print(f"bf16 head vs bf16 oracle {err:.2e}, vs fp32 oracle {gap:.2e}")
    assert gap > 3 * err, (gap, err)


@pytest.mark.parametrize("env,n,B,block,scale,layers", [
    ("cartpole", 2048, 512, 3, 4, 2),
    ("cartpole", 64, 64, 1, 4, 2),       # the smallest minibatch: split kernel, one split
    ("cartpole_continuous", 2048, 1024, 1, 4, 2),
    ("voxelnav16", 1024, 512, 2, 4, 2),
    ("cartpole", 4096, 4096, 1, 4, 2),   # fused weight gradients over 4096 rows
    ("cartpole", 6144, 6144, 0, 1, 2),   # 64 tiles of 32x32: split kernel, 16 splits of 384 rows
    ("cartpole", 1024, 512, 1, 8, 2),    # hidden 1024 (512 tiles, fused)
    ("cartpole", 1024, 512, 1, 1, 8),    # 8 blocks (256 tiles, fused)
    ("cartpole", 1024, 512, 0, 8, 8),    # the largest policy: 2048 tiles, split kernel
])
def test_bf16_minibatch(mg, orc, env, n, B, block, scale, layers):
    """One PPO minibatch in bf16 mode against the oracle's bf16 train step on
    the GPU's own rollout: recomputed head (median/p99/max), the Adam first
    moment (0.1 x the clipped gradient) per parameter group, post-Adam weights
    and LossStats."""
    from parity import TOL_TRAIN, assert_close
    from test_gpu_train import block_rows, group_errors

    eid, kernel = ENVS[env]
    T = 2
    gym = mg.Gym(kernel, n, 0)
    model = mg.PPOModel(gym, scale=scale, layers=layers, horizon=T, minibatch=B, precision="bf16")
    d = orc.dims(eid, hidden=128 * scale, layers=layers, bf16=True)
    model.collect()
    s = model.download_slots()
    p0 = model.params()
    model.train_block(block)
    hp = orc.hparams()
    P, M, V = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    st, grad, head = orc.train_minibatch(d, hp, P, M, V, 1, *block_rows(s, n, B, block), threads=THREADS)
    assert_close_bf16(model.head(), head, "recomputed head")
    m1, _, _ = model.adam_state()
    errs = group_errors(model.pv, m1, M)
    print("bf16 moment, gpu vs oracle per group:", errs)
    assert max(errs.values()) < 1e-2, errs
    # the same gradient computed in fp32 is much further away
    P2, M2, V2 = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    orc.train_minibatch(orc.dims(eid, hidden=128 * scale, layers=layers), hp, P2, M2, V2, 1,
                        *block_rows(s, n, B, block), threads=THREADS)
    e32 = group_errors(model.pv, M2, M)
    assert e32["up0"] > 3 * errs["up0"], (e32["up0"], errs["up0"])
    assert_close(model.params(), P, TOL_TRAIN, "post-Adam weights")
    got, want = np.array(model.last_stats().as_tuple()), np.array(st.as_tuple())
    assert_close(got[[0, 1, 2, 3, 5]], want[[0, 1, 2, 3, 5]], TOL_TRAIN, "LossStats")


def test_bf16_full_loop_learns(mg):
    """CartPole trained in bf16 mode improves its mean episode length."""
    gym = mg.Gym("rollout_cartpole", 4096, 0)
    model = mg.PPOModel(gym, horizon=32, precision="bf16")
    lens = []
    for it in range(12):
        model.collect()
        d = model.download_slots()["done"]
        lens.append(d.size / max(1, d.sum()))
        model.train(4)
        assert np.all(np.isfinite(model.last_stats().as_tuple()))
    assert np.mean(lens[-3:]) > 1.5 * np.mean(lens[:3]), lens


@pytest.mark.parametrize("env", ["cartpole", "cartpole_continuous"])
def test_bf16_train_epochs(mg, orc, env):
    """train(2) in bf16 mode over 2 slots x 2 blocks against the oracle's bf16
    train loop: the same block order, every minibatch's LossStats and the
    weights after 2 epochs within 1e-3. The clip fraction counts rows with
    |ratio - 1| > clip; bf16 rounding flips move about 1% of head values by
    more than 1e-5, so up to 1% of the rows (at least 2) may sit on the other
    side of the clip boundary."""
    import ctypes as C

    from parity import TOL_TRAIN, assert_close

    n, T, B = 1024, 2, 512
    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, n, 7)
    model = mg.PPOModel(gym, horizon=T, seed=7, minibatch=B, precision="bf16")
    d = orc.dims(eid, bf16=True)
    model.collect()
    s = model.download_slots()
    p0 = model.params()
    model.train(2)
    stats = model.train_stats()
    P, M, V = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    step, shuf = C.c_uint32(0), C.c_uint64(0)
    orc.lib().orc_shuffle_state_init(7, C.byref(shuf))
    blocks = T * (n // B)
    order = np.arange(blocks, dtype=np.uint32)
    ost = (orc.Stats * (2 * blocks))()
    orc.lib().orc_train(C.byref(d), C.byref(orc.hparams()), orc.ptr(P), orc.ptr(M), orc.ptr(V), C.byref(step),
                        C.byref(shuf), n, T, B, 2, orc.ptr(np.ascontiguousarray(s["obs"])),
                        orc.ptr(np.ascontiguousarray(s["actions"])), orc.ptr(np.ascontiguousarray(s["adv"])),
                        orc.ptr(np.ascontiguousarray(s["ret"])), orc.ptr(np.ascontiguousarray(s["logp"])), ost,
                        orc.ptr(order), THREADS)
    assert list(model.last_order()[-blocks:]) == list(order)
    ostats = np.array([ost[i].as_tuple() for i in range(2 * blocks)], np.float32)
    cols = [0, 1, 2, 3, 5]
    assert_close(stats[:, cols], ostats[:, cols], TOL_TRAIN, "per-minibatch LossStats")
    assert np.all(np.abs(stats[:, 4] - ostats[:, 4]) * B <= max(2, B // 100) + 1e-3), (stats[:, 4], ostats[:, 4])
    assert_close(model.params(), P, TOL_TRAIN, "weights after 2 epochs")
