"""mg_ppo_train_block_noalloc (the minibatch update for callers that cannot
allocate: its workspace is the library's static device array) against
mg_ppo_train_block on identical models: two calls in a row, the second with a
smaller minibatch (and the Gaussian head, whose tile partials include the
arena padding after log_std), so the second runs on the array the first left
behind. Both run the same kernels on the same inputs, so parameters, Adam
moments, the recomputed head and the LossStats must agree bit for bit, and the
no-alloc model ends without a train workspace of its own (its captures query
still reports that none was bound). A policy whose workspace exceeds the array
is rejected before any launch."""
import numpy as np
import pytest

from parity import ENVS, assert_bit_exact

pytestmark = pytest.mark.gpu


def twin_models(mg, env, n, B, seed, scale=4):
    _, kernel = ENVS[env]
    out = []
    for _ in range(2):
        gym = mg.Gym(kernel, n, seed)
        model = mg.PPOModel(gym, horizon=2, seed=seed, minibatch=B, scale=scale)
        model.collect()
        out.append((gym, model))
    return out


def test_noalloc_matches_train_block(mg):
    from metalgym_amd._capi import CapiError

    for env, n, B, block, seed in (("cartpole", 4096, 4096, 1, 3), ("cartpole_continuous", 1024, 512, 2, 5)):
        print(f"case {env} n={n} B={B} block={block}", flush=True)
        (_, ref), (gym, na) = twin_models(mg, env, n, B, seed)
        assert_bit_exact(na.params(), ref.params(), f"{env} initial parameters")
        ref.train_block(block)
        stats = mg.DeviceBuffer(6 * 4)
        na.train_block_noalloc(block, stats.ptr)
        gym.sync()
        assert_bit_exact(na.params(), ref.params(), f"{env} parameters")
        (m_na, v_na, s_na), (m_ref, v_ref, s_ref) = na.adam_state(), ref.adam_state()
        assert s_na == s_ref == 1
        assert_bit_exact(m_na, m_ref, f"{env} Adam m")
        assert_bit_exact(v_na, v_ref, f"{env} Adam v")
        assert_bit_exact(na.head(), ref.head(), f"{env} recomputed head")
        got = stats.download(np.float32, (6,))
        want = np.array(ref.last_stats().as_tuple(), np.float32)
        assert_bit_exact(got, want, f"{env} LossStats")
        # stats_out NULL: the LossStats stay in the array; the update is the same
        na.train_block_noalloc(block)
        ref.train_block(block)
        gym.sync()
        assert_bit_exact(na.params(), ref.params(), f"{env} parameters after a second step")
        # the no-alloc model never bound a workspace of its own: nothing was allocated
        with pytest.raises(CapiError) as e:
            na.train_capture(0)
        assert e.value.rc == -5, e.value


def test_noalloc_rejects_a_workspace_beyond_the_array(mg):
    from metalgym_amd._capi import CapiError

    (_, _), (gym, model) = twin_models(mg, "cartpole", 4096, 4096, 0, scale=8)  # hidden 1024: 108 MiB
    p0 = model.params()
    with pytest.raises(CapiError) as e:
        model.train_block_noalloc(0)
    assert e.value.rc == -1 and "static scratch" in str(e.value)
    gym.sync()
    assert_bit_exact(model.params(), p0, "parameters after the rejected call")
