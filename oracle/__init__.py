"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (oracle/oracle.h).

Imported by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
leg, where it is the checker (or the timed CPU baseline). The product package
metalgym_amd never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

CARTPOLE, CARTPOLE_CONT, CARTPOLE_CONT_CLAMP, VOXELNAV16, VOXELNAV = 0, 1, 2, 3, 4
ENV_KERNELS = {
    CARTPOLE: "rollout_cartpole",
    CARTPOLE_CONT: "rollout_cartpole_continuous",
    CARTPOLE_CONT_CLAMP: "rollout_cartpole_continuous_clamp",
    VOXELNAV16: "rollout_voxelnav16",
    VOXELNAV: "rollout_voxelnav",
}


class EnvInfo(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("state_bytes", "action_bytes", "obs_dim", "act_dim", "continuous")]


class Dims(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("obs_dim", "act_dim", "embed", "hidden", "layers", "continuous", "bf16")]


class Layout(C.Structure):
    _fields_ = [
        ("count", C.c_uint32),
        ("float_group", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("off_in_w", C.c_uint32),
        ("off_in_b", C.c_uint32),
        ("off_ln_gamma", C.c_uint32 * 9),
        ("off_ln_beta", C.c_uint32 * 9),
        ("off_up", C.c_uint32 * 8),
        ("off_down", C.c_uint32 * 8),
        ("off_head", C.c_uint32),
        ("off_log_std", C.c_uint32),
    ]


class HParams(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("clip", "value_coef", "entropy_coef", "max_grad_norm", "gamma", "lambda_", "lr")]


class Stats(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("policy", "value", "entropy", "approx_kl", "clip_frac", "grad_norm")]

    def as_tuple(self):
        return tuple(getattr(self, n) for n, _ in self._fields_)


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def _signatures():
    P = C.c_void_p
    u32, f32 = C.c_uint32, C.c_float
    return {
        "orc_rng_next": (u32, [P]),
        "orc_rng_uniform": (f32, [P]),
        "orc_rng_uniform_range": (f32, [P, f32, f32]),
        "orc_rng_int": (u32, [P, u32]),
        "orc_gym_init": (None, [C.c_int, u32, u32, P, P, P, P]),
        "orc_env_info_get": (C.c_int, [C.c_int, P]),
        "orc_env_reset": (None, [C.c_int, P, P]),
        "orc_env_step": (None, [C.c_int, P, P, P, P, P]),
        "orc_rollout": (None, [C.c_int, u32, u32, C.c_int, P, P, P, P, P, P, P, P, C.c_int]),
        "orc_round_bf16": (f32, [f32]),
        "orc_expf": (f32, [f32]),
        "orc_logf": (f32, [f32]),
        "orc_sinf": (f32, [f32]),
        "orc_cosf": (f32, [f32]),
        "orc_tanhf": (f32, [f32]),
        "orc_layout_get": (C.c_int, [P, P]),
        "orc_init_params": (None, [P, u32, P]),
        "orc_splitmix_next": (C.c_uint64, [P]),
        "orc_forward": (None, [P, P, P, u32, P, C.c_int]),
        "orc_sample": (None, [P, P, P, u32, P, P, P, P]),
        "orc_gae": (None, [P, P, P, P, u32, u32, u32, u32, f32, f32, P, P]),
        "orc_collect": (None, [C.c_int, P, P, u32, u32, C.c_int, f32, f32] + [P] * 14 + [C.c_int]),
        "orc_train_minibatch": (None, [P, P, P, P, P, u32, u32, P, P, P, P, P, P, P, P, C.c_int]),
        "orc_train_minibatch_masked": (None, [P, P, P, P, P, u32, u32, P, P, P, P, P, P, P, P, P, P, C.c_int]),
        "orc_shuffle_state_init": (None, [u32, P]),
        "orc_shuffle_blocks": (None, [P, P, u32]),
        "orc_train": (None, [P, P, P, P, P, P, P, u32, u32, u32, u32, P, P, P, P, P, P, P, C.c_int]),
    }


def load(path: str):
    """Load an oracle build and declare its signatures."""
    L = C.CDLL(path)
    for name, (res, args) in _signatures().items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def lib():
    """The oracle library. MG_ORACLE_LIB names another build of oracle.cpp
    (the mutation tests load deliberately broken copies this way); by default
    the in-tree build, made on first use."""
    global _lib
    if _lib is None:
        path = os.environ.get("MG_ORACLE_LIB") or LIB_PATH
        if path == LIB_PATH and not os.path.exists(LIB_PATH):
            build()
        _lib = load(path)
    return _lib


def ptr(a):
    """Raw pointer of a numpy array (or None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def env_info(env: int) -> EnvInfo:
    info = EnvInfo()
    lib().orc_env_info_get(env, C.byref(info))
    return info


def dims(env: int, hidden: int = 512, layers: int = 2, embed: int = 128, bf16: bool = False) -> Dims:
    i = env_info(env)
    return Dims(i.obs_dim, i.act_dim, embed, hidden, layers, i.continuous, 1 if bf16 else 0)


def layout(d: Dims) -> Layout:
    L = Layout()
    lib().orc_layout_get(C.byref(d), C.byref(L))
    return L


def action_dtype(env: int):
    return np.float32 if env_info(env).continuous else np.int32


def action_shape(env: int, *lead):
    i = env_info(env)
    return tuple(lead) + ((i.act_dim,) if i.continuous else ())


class GymState:
    """Host copy of a gym's live buffers, laid out like the device buffers."""

    def __init__(self, env: int, n: int, seed: int = 0):
        i = env_info(env)
        self.env, self.n, self.info = env, n, i
        self.state = np.zeros(n * i.state_bytes, np.uint8)
        self.rng = np.zeros(n, np.uint32)
        self.done = np.zeros(n, np.uint8)
        self.actions = np.zeros(action_shape(env, n), action_dtype(env))
        lib().orc_gym_init(env, n, seed, ptr(self.state), ptr(self.rng), ptr(self.done), ptr(self.actions))

    def copy(self):
        g = GymState.__new__(GymState)
        g.env, g.n, g.info = self.env, self.n, self.info
        g.state, g.rng, g.done, g.actions = self.state.copy(), self.rng.copy(), self.done.copy(), self.actions.copy()
        return g


def rollout(g: GymState, steps: int, random: bool = True, actions_in=None, threads: int = 8):
    n, i = g.n, g.info
    acts = np.zeros(action_shape(g.env, steps, n), action_dtype(g.env))
    obs = np.zeros((steps, n, i.obs_dim), np.float32)
    rew = np.zeros((steps, n), np.float32)
    dn = np.zeros((steps, n), np.uint8)
    if not random:
        acts = np.ascontiguousarray(actions_in, dtype=action_dtype(g.env)).reshape(acts.shape)
    lib().orc_rollout(g.env, n, steps, 1 if random else 0, ptr(g.state), ptr(g.rng), ptr(g.done),
                      None if random else ptr(acts), ptr(acts) if random else None, ptr(obs), ptr(rew), ptr(dn),
                      threads)
    return acts, obs, rew, dn


def init_params(d: Dims, seed: int = 0) -> np.ndarray:
    p = np.zeros(layout(d).count, np.float32)
    lib().orc_init_params(C.byref(d), seed, ptr(p))
    return p


def forward(d: Dims, params, obs, threads: int = 8):
    obs = np.ascontiguousarray(obs, np.float32)
    rows = obs.shape[0]
    head = np.zeros((rows, d.act_dim + 1), np.float32)
    lib().orc_forward(C.byref(d), ptr(params), ptr(obs), rows, ptr(head), threads)
    return head


def gae(reward, done, value, head, act_dim, gamma=0.99, lam=0.95):
    T, n = reward.shape
    adv = np.zeros((T, n), np.float32)
    ret = np.zeros((T, n), np.float32)
    head = np.ascontiguousarray(head, np.float32)
    lib().orc_gae(ptr(np.ascontiguousarray(reward, np.float32)), ptr(np.ascontiguousarray(done, np.uint8)),
                  ptr(np.ascontiguousarray(value, np.float32)), ptr(head), head.shape[1], act_dim, n, T, gamma, lam,
                  ptr(adv), ptr(ret))
    return adv, ret


class Slots:
    def __init__(self, env: int, n: int, T: int):
        i = env_info(env)
        self.obs = np.zeros((T + 1, n, i.obs_dim), np.float32)
        self.actions = np.zeros(action_shape(env, T, n), action_dtype(env))
        self.logp = np.zeros((T, n), np.float32)
        self.value = np.zeros((T, n), np.float32)
        self.reward = np.zeros((T, n), np.float32)
        self.done = np.zeros((T, n), np.uint8)
        self.adv = np.zeros((T, n), np.float32)
        self.ret = np.zeros((T, n), np.float32)
        self.head = np.zeros((n, i.act_dim + 1), np.float32)


def collect(g: GymState, d: Dims, params, T: int, slots: Slots, first: bool, gamma=0.99, lam=0.95,
            teacher_actions=None, threads: int = 8):
    sampled = np.zeros_like(slots.actions)
    ta = None if teacher_actions is None else np.ascontiguousarray(teacher_actions, action_dtype(g.env))
    lib().orc_collect(g.env, C.byref(d), ptr(params), g.n, T, 1 if first else 0, gamma, lam, ptr(g.state), ptr(g.rng),
                      ptr(g.done), ptr(slots.obs), ptr(slots.actions), ptr(slots.logp), ptr(slots.value),
                      ptr(slots.reward), ptr(slots.done), ptr(slots.adv), ptr(slots.ret), ptr(slots.head), ptr(ta),
                      ptr(sampled), threads)
    return sampled


def hparams(clip=0.2, value_coef=0.5, entropy_coef=0.01, max_grad_norm=0.5, gamma=0.99, lam=0.95, lr=3e-4):
    return HParams(clip, value_coef, entropy_coef, max_grad_norm, gamma, lam, lr)


def train_minibatch(d: Dims, hp: HParams, params, m, v, step, obs, actions, adv, ret, old_logp, threads: int = 8):
    """One minibatch update in place; returns (stats, grad, head)."""
    rows = obs.shape[0]
    grad = np.zeros_like(params)
    head = np.zeros((rows, d.act_dim + 1), np.float32)
    st = Stats()
    lib().orc_train_minibatch(C.byref(d), C.byref(hp), ptr(params), ptr(m), ptr(v), step, rows,
                              ptr(np.ascontiguousarray(obs, np.float32)), ptr(np.ascontiguousarray(actions)),
                              ptr(np.ascontiguousarray(adv, np.float32)), ptr(np.ascontiguousarray(ret, np.float32)),
                              ptr(np.ascontiguousarray(old_logp, np.float32)), ptr(grad), C.byref(st), ptr(head),
                              threads)
    return st, grad, head


def train_minibatch_masked(d: Dims, hp: HParams, params, m, v, step, obs, actions, adv, ret, old_logp, relu_mask,
                           threads: int = 8):
    """train_minibatch with the forward's ReLU decisions given (relu_mask
    [rows][layers][hidden], bool or uint8; None keeps z > 0); returns (stats,
    grad, head, preact) with the pre-activations [rows][layers][hidden]."""
    rows = obs.shape[0]
    grad = np.zeros_like(params)
    head = np.zeros((rows, d.act_dim + 1), np.float32)
    preact = np.zeros((rows, d.layers, d.hidden), np.float32)
    mask = None if relu_mask is None else np.ascontiguousarray(relu_mask, np.uint8)
    if mask is not None:
        assert mask.shape == preact.shape, (mask.shape, preact.shape)
    st = Stats()
    lib().orc_train_minibatch_masked(C.byref(d), C.byref(hp), ptr(params), ptr(m), ptr(v), step, rows,
                                     ptr(np.ascontiguousarray(obs, np.float32)), ptr(np.ascontiguousarray(actions)),
                                     ptr(np.ascontiguousarray(adv, np.float32)),
                                     ptr(np.ascontiguousarray(ret, np.float32)),
                                     ptr(np.ascontiguousarray(old_logp, np.float32)), ptr(grad), C.byref(st),
                                     ptr(head), ptr(mask), ptr(preact), threads)
    return st, grad, head, preact
