"""The C ABI library loads, exports every declared entry point, registers the
built-in envs and rejects bad configurations, all without touching a GPU."""
import ctypes as C
import os
import re

import pytest

from metalgym_amd._capi import PPOConfig

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include", "mg")):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", "mg", fn)).read()
        if 'extern "C"' not in text:
            continue
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mg_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_every_declared_symbol_is_exported(mg):
    names = declared_functions()
    assert len(names) > 40
    lib = C.CDLL(mg.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version(mg):
    assert mg.lib().mg_abi_version() == 4


def test_builtin_envs_registered(mg):
    names = mg.env_names()
    for k in ("rollout_cartpole", "rollout_cartpole_continuous", "rollout_cartpole_continuous_clamp",
              "rollout_voxelnav16"):
        assert k in names


def test_env_descriptors(mg):
    from metalgym_amd._capi import env_desc

    d = env_desc("rollout_cartpole")
    assert (d.state_bytes, d.action_bytes, d.obs_dim, d.act_dim, d.continuous, d.state_in_registers) == (20, 4, 4, 2,
                                                                                                          0, 1)
    d = env_desc("rollout_cartpole_continuous")
    assert (d.action_bytes, d.act_dim, d.continuous) == (4, 1, 1)
    d = env_desc("rollout_voxelnav16")
    assert (d.obs_dim, d.act_dim, d.state_in_registers) == (30, 6, 0)
    assert d.state_bytes == 32 + 4096


def test_unknown_env_is_not_found(mg):
    h = C.c_void_p()
    rc = mg.lib().mg_gym_create(b"rollout_nope", 64, 0, C.byref(h))
    assert rc == -2 and h.value is None
    assert b"rollout_nope" in mg.lib().mg_last_error()


def test_gym_rejects_zero_envs(mg):
    h = C.c_void_p()
    assert mg.lib().mg_gym_create(b"rollout_cartpole", 0, 0, C.byref(h)) == -1


def cfg(**kw):
    base = dict(embed=128, scale=4, layers=2, horizon=32, minibatch=0, seed=0, lr=3e-4, precision=0)
    base.update(kw)
    return PPOConfig(**base)


def test_valid_config_passes(mg):
    assert mg.lib().mg_ppo_check_config(b"rollout_cartpole", 4096, C.byref(cfg())) == 0
    assert mg.lib().mg_ppo_check_config(b"rollout_voxelnav16", 262144, C.byref(cfg())) == 0
    # the largest minibatch whose captures keep 32-bit offsets at hidden 1024
    assert mg.lib().mg_ppo_check_config(b"rollout_cartpole", 262144, C.byref(cfg(minibatch=262144, scale=8))) == 0


# model/ppo.h:290-298: every constructor validation failure, forced from the host
@pytest.mark.parametrize("n,kw,needle", [
    (4000, {}, b"multiple of 64"),
    (4096, dict(embed=64), b"embedDim"),
    (4096, dict(layers=0), b"layers"),
    (4096, dict(layers=9), b"layers"),
    (4096, dict(horizon=0), b"horizon"),
    (4096, dict(scale=0), b"scale"),
    (4096, dict(minibatch=100), b"minibatch"),
    (4096, dict(minibatch=8192), b"minibatch"),
    (524288, dict(minibatch=524288, scale=8), b"31 bits"),  # captures of 2 GiB: beyond 32-bit offsets
])
def test_config_validation(mg, n, kw, needle):
    rc = mg.lib().mg_ppo_check_config(b"rollout_cartpole", n, C.byref(cfg(**kw)))
    assert rc == -1
    assert needle in mg.lib().mg_last_error()


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    import metalgym_amd._capi as capi

    monkeypatch.setattr(capi, "_lib", None)
    monkeypatch.setattr(capi, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="no fallback"):
        capi.lib()
