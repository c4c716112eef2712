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
