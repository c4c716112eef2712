"""collect() on the GPU against the oracle, teacher-forced per step: the
oracle replays every env with the GPU's actions, so RNG streams, env state,
resets and done flags must match bit for bit, the policy head and values to
1e-4, and GAE bit for bit on the GPU's own inputs (model/ppo.h:716-751)."""
import numpy as np
import pytest

from parity import ENVS, THREADS, TOL_HEAD, assert_bit_exact, assert_close, assert_close_bf16

pytestmark = pytest.mark.gpu


def run_collect_parity(mg, orc, env, n, T, layers=2, scale=4, seed=0, collects=2, bf16=False):
    close = (lambda g, w, what: assert_close_bf16(g, w, what)) if bf16 else \
        (lambda g, w, what: assert_close(g, w, TOL_HEAD, what))
    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, n, seed)
    model = mg.PPOModel(gym, scale=scale, layers=layers, horizon=T, seed=seed, precision="bf16" if bf16 else "fp32")
    d = orc.dims(eid, hidden=128 * scale, layers=layers, bf16=bf16)
    params = orc.init_params(d, seed)
    assert_bit_exact(model.params(), params, "initial parameters")
    g = orc.GymState(eid, n, seed)
    slots = orc.Slots(eid, n, T)
    for c in range(collects):
        model.collect()
        s = model.download_slots()
        head = model.head()
        sampled = orc.collect(g, d, params, T, slots, first=(c == 0), teacher_actions=s["actions"],
                              threads=THREADS)
        tag = f"{env} collect {c}"
        # env side: bit-exact under teacher forcing
        assert_bit_exact(s["obs"], slots.obs, f"{tag} obs slots")
        assert_bit_exact(s["reward"], slots.reward, f"{tag} rewards")
        assert_bit_exact(s["done"], slots.done, f"{tag} dones")
        assert_bit_exact(gym.rng(), g.rng, f"{tag} rng")
        assert_bit_exact(gym.state(), g.state, f"{tag} state")
        assert_bit_exact(gym.done(), g.done, f"{tag} live done")
        # policy side: within 1e-4 (bf16: in bulk, with bounded flipped rows)
        close(s["value"], slots.value, f"{tag} values")
        close(s["logp"], slots.logp, f"{tag} logp")
        close(head, slots.head, f"{tag} bootstrap head")
        if gym.continuous:
            close(s["actions"], sampled, f"{tag} gaussian samples")
        else:
            flips = int((s["actions"] != sampled).sum())
            assert flips <= max(2, s["actions"].size // (1000 if bf16 else 10000)), f"{tag}: {flips} sampled actions differ"
        # GAE: bit-exact on the GPU's own inputs, 1e-4 against the oracle's
        adv, ret = orc.gae(s["reward"], s["done"], s["value"], head, gym.act_dim)
        assert_bit_exact(s["adv"], adv, f"{tag} advantages")
        assert_bit_exact(s["ret"], ret, f"{tag} returns")
        close(s["adv"], slots.adv, f"{tag} advantages vs oracle")
    return model, s


@pytest.mark.parametrize("env,n,T", [
    ("cartpole", 4096, 8),
    ("cartpole", 64, 1),         # the fewest envs (four 16-row tiles), one step
    ("cartpole", 192, 3),
    ("cartpole", 64 * 576, 2),   # 64-row tiles (n >= 64 * 512)
    ("cartpole_continuous", 2048, 8),
    ("cartpole_continuous_clamp", 2048, 8),
    ("voxelnav16", 1024, 8),
    ("voxelnav", 1024, 8),       # heightmaps staged in LDS: 16-row tiles
    ("voxelnav", 8192, 2),       # 32-row tiles, heightmaps in LDS (256 workgroups)
    ("voxelnav", 16384, 2),      # 32-row tiles, heightmaps in device memory, two workgroups per CU
    ("voxelnav", 32768, 2),      # 64-row tiles, the same
])
def test_collect_teacher_forced(mg, orc, env, n, T):
    run_collect_parity(mg, orc, env, n, T)


@pytest.mark.parametrize("env,n,block", [
    ("cartpole", 262144, 37),              # config 2 (the headline) and config 3
    ("cartpole_continuous", 65536, 21),    # config 4
    ("cartpole_continuous", 262144, 1999),
    ("voxelnav16", 262144, 1000),          # config 5
])
def test_collect_full_size_subset(mg, orc, env, n, block):
    """A benchmarked configuration at its full size (T = 32): two collects on
    the GPU; the oracle replays 1536 of the envs (first, last, tile edges and a
    random spread) teacher-forced from the same seeds. Envs are independent, so
    the subset must match bit for bit (values 1e-4); GAE is checked bit for
    bit over all envs on the GPU's own inputs. Then one 4096-row minibatch of
    the full-size rollout (the benchmark's minibatch shape) against the
    oracle's train step, with the GPU's ReLU decisions replayed."""
    from parity import check_minibatch
    from test_gpu_train import block_rows

    eid, kernel = ENVS[env]
    T, B = 32, 4096
    gym = mg.Gym(kernel, n, 0)
    model = mg.PPOModel(gym, horizon=T)
    d = orc.dims(eid)
    params = orc.init_params(d, 0)
    rs = np.random.default_rng(17)
    idx = np.unique(np.concatenate([[0, 1, 63, 64, n // 2, n - 65, n - 1], rs.choice(n, 1529, replace=False)]))
    full = orc.GymState(eid, n, 0)
    g = orc.GymState(eid, idx.size, 0)
    sb = full.info.state_bytes
    g.state[:] = full.state.reshape(n, sb)[idx].ravel()
    g.rng[:] = full.rng[idx]
    g.done[:] = full.done[idx]
    del full
    slots = orc.Slots(eid, idx.size, T)
    for c in range(2):
        model.collect()
        s = model.download_slots()
        head = model.head()
        orc.collect(g, d, params, T, slots, first=(c == 0), teacher_actions=s["actions"][:, idx], threads=THREADS)
        tag = f"{n}-env {env} collect {c}"
        assert_bit_exact(s["obs"][:, idx], slots.obs, f"{tag} obs slots")
        assert_bit_exact(s["reward"][:, idx], slots.reward, f"{tag} rewards")
        assert_bit_exact(s["done"][:, idx], slots.done, f"{tag} dones")
        assert_bit_exact(gym.rng()[idx], g.rng, f"{tag} rng")
        assert_bit_exact(gym.state().reshape(n, sb)[idx].ravel(), g.state, f"{tag} state")
        assert_close(s["value"][:, idx], slots.value, TOL_HEAD, f"{tag} values")
        assert_close(s["logp"][:, idx], slots.logp, TOL_HEAD, f"{tag} logp")
        assert_close(head[idx], slots.head, TOL_HEAD, f"{tag} bootstrap head")
        adv, ret = orc.gae(s["reward"], s["done"], s["value"], head, gym.act_dim)
        assert_bit_exact(s["adv"], adv, f"{tag} advantages")
        assert_bit_exact(s["ret"], ret, f"{tag} returns")
    assert np.isfinite(s["value"]).all() and np.isfinite(s["logp"]).all()
    p0 = model.params()
    model.train_block(block)
    check_minibatch(model, orc, d, orc.hparams(), p0, block_rows(s, n, B, block), B)


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_collect_and_forward_after_train(mg, orc, precision):
    """train() rewrites only the weight copies its own row pass reads; collect
    (64-row tiles here, which read the 32-wide copies) and forward() after it
    must see the trained weights. The oracle continues from the GPU's env
    state after the first collect and replays the second one teacher-forced
    with the post-train parameters."""
    bf16 = precision == "bf16"
    close = (lambda g, w, what: assert_close_bf16(g, w, what)) if bf16 else \
        (lambda g, w, what: assert_close(g, w, TOL_HEAD, what))
    eid, kernel = ENVS["cartpole"]
    n, T = 64 * 512, 2
    gym = mg.Gym(kernel, n, 0)
    model = mg.PPOModel(gym, horizon=T, precision=precision)
    d = orc.dims(eid, bf16=bf16)
    model.collect()
    s = model.download_slots()
    g = orc.GymState(eid, n, 0)
    g.state[:] = gym.state()
    g.rng[:] = gym.rng()
    g.done[:] = gym.done()
    slots = orc.Slots(eid, n, T)
    slots.obs[:] = s["obs"]
    p0 = model.params()
    model.train(1)
    p1 = model.params()
    assert np.abs(p1 - p0).max() > 1e-6, "training left the weights unchanged"
    model.collect()
    s = model.download_slots()
    orc.collect(g, d, p1, T, slots, first=False, teacher_actions=s["actions"], threads=THREADS)
    assert_bit_exact(s["obs"], slots.obs, "obs slots after train")
    close(s["value"], slots.value, "values after train")
    close(s["logp"], slots.logp, "logp after train")
    close(model.head(), slots.head, "bootstrap head after train")
    model.train(1)
    rs = np.random.default_rng(9)
    obs = (rs.standard_normal((4096, gym.obs_dim)) * 2).astype(np.float32)
    close(model.forward(obs), orc.forward(d, model.params(), obs, threads=THREADS), "forward after train")


@pytest.mark.parametrize("n,T,layers,scale", [
    (1024, 4, 1, 1),
    (1024, 4, 3, 2),
    (1024, 2, 8, 1),     # the most blocks (MG_MAX_LAYERS), 16-row tiles
    (1024, 2, 2, 8),     # the widest hidden layer (1024), 16-row tiles
    (8192, 2, 2, 8),     # 32-row tiles
    (32768, 2, 8, 1),    # 64-row tiles; 9 LNs: small parameters read from the arena, not LDS
])
def test_collect_other_shapes(mg, orc, n, T, layers, scale):
    run_collect_parity(mg, orc, "cartpole", n, T, layers=layers, scale=scale, seed=11, collects=1)


@pytest.mark.parametrize("env", ["cartpole", "voxelnav16", "cartpole_continuous"])
def test_forward_matches_oracle(mg, orc, env):
    """forward() (model/ppo.h:628-634) on arbitrary rows, including a ragged count."""
    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, 256, 0)
    model = mg.PPOModel(gym, horizon=4)
    d = orc.dims(eid)
    rs = np.random.default_rng(3)
    obs = (rs.standard_normal((1000, gym.obs_dim)) * 3).astype(np.float32)
    head = model.forward(obs)
    want = orc.forward(d, model.params(), obs, threads=THREADS)
    assert_close(head, want, TOL_HEAD, "head")


@pytest.mark.parametrize("env", ["cartpole", "voxelnav16", "cartpole_continuous"])
def test_sampler_matches_oracle(mg, orc, env):
    """Sampling alone on a given head: actions and RNG bit-exact, logp to 1e-4."""
    import ctypes as C

    eid, kernel = ENVS[env]
    gym = mg.Gym(kernel, 256, 0)
    model = mg.PPOModel(gym, horizon=4)
    d = orc.dims(eid)
    rs = np.random.default_rng(4)
    rows = 4096
    head = rs.standard_normal((rows, gym.act_dim + 1)).astype(np.float32)
    rng = rs.integers(1, 2**32 - 1, rows, dtype=np.uint32)
    a, lp, v, r2 = model.sample(head, rng)
    oa = np.zeros(gym.action_shape(rows), gym.action_dtype)
    olp = np.zeros(rows, np.float32)
    ov = np.zeros(rows, np.float32)
    orng = rng.copy()
    orc.lib().orc_sample(C.byref(d), orc.ptr(model.params()), orc.ptr(head), rows, orc.ptr(orng), orc.ptr(oa),
                         orc.ptr(olp), orc.ptr(ov))
    assert_bit_exact(r2, orng, "rng")
    assert_bit_exact(a, oa, "actions")
    assert_bit_exact(lp, olp, "logp")
    assert_bit_exact(v, ov, "value")
