"""ctypes binding of include/mg/capi.h (see the package docstring)."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmetalgym_amd.so")

MAX_LAYERS = 8
K_NAMES = ["rollout", "collect", "gae", "adv_stats", "train_rows", "train_dw", "grad_reduce", "adam", "forward",
           "copy"]


class CapiError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"[{rc}] {msg}")
        self.rc = rc


P = C.c_void_p
u32, f32 = C.c_uint32, C.c_float


class EnvDesc(C.Structure):
    _fields_ = [(n, u32) for n in ("abi_version", "state_bytes", "action_bytes", "obs_dim", "act_dim", "continuous",
                                   "state_in_registers", "reserved")] + [("kernel", C.c_char_p), ("rollout", P),
                                                                         ("collect", P)]


class PolicyView(C.Structure):
    _fields_ = [(n, P) for n in ("params", "frag_fwd32", "frag_fwd16", "frag_bwd16", "frag_fwd32_bf",
                                 "frag_fwd16_bf", "frag_bwd16_bf")] + [(n, u32) for n in (
        "obs_dim", "act_dim", "embed", "hidden", "layers", "head_dim", "continuous", "precision", "count", "off_in_w",
        "off_in_b")] + [
        ("off_ln_gamma", u32 * (MAX_LAYERS + 1)),
        ("off_ln_beta", u32 * (MAX_LAYERS + 1)),
        ("off_up", u32 * MAX_LAYERS),
        ("off_down", u32 * MAX_LAYERS),
        ("off_head", u32),
        ("off_log_std", u32),
        ("float_group", u32),
    ]


class CollectArgs(C.Structure):
    """mg_collect_args: the launch arguments of an env's fused collect kernel."""
    _fields_ = [("stream", P), ("policy", PolicyView), ("n", u32), ("horizon", u32), ("first", u32),
                ("reserved", u32), ("state", P), ("rng", P), ("done", P), ("obs_slots", P), ("action_slots", P),
                ("logp_slots", P), ("value_slots", P), ("reward_slots", P), ("done_slots", P), ("head_out", P)]


COLLECT_FN = C.CFUNCTYPE(C.c_int, C.POINTER(CollectArgs))


class GymBuffers(C.Structure):
    _fields_ = [("stream", P), ("env", C.POINTER(EnvDesc)), ("n", u32), ("seed", u32), ("state", P), ("actions", P),
                ("obs", P), ("reward", P), ("done", P), ("rng", P)]


class PPOConfig(C.Structure):
    _fields_ = [(n, u32) for n in ("embed", "scale", "layers", "horizon", "minibatch", "seed")] + [("lr", f32),
                                                                                                    ("precision", u32)]


class PPOHParams(C.Structure):
    _fields_ = [(n, f32) for n in ("clip", "value_coef", "entropy_coef", "max_grad_norm", "gamma", "lambda_")]


class LossStats(C.Structure):
    _fields_ = [(n, f32) for n in ("policy", "value", "entropy", "approx_kl", "clip_frac", "grad_norm")]

    def as_tuple(self):
        return tuple(getattr(self, n) for n, _ in self._fields_)


class PPOSlots(C.Structure):
    _fields_ = [(n, P) for n in ("obs", "actions", "logp", "value", "reward", "done", "advantage", "ret")] + [
        ("n", u32), ("horizon", u32)]


class KernelTimes(C.Structure):
    _fields_ = [("total_ms", C.c_double * len(K_NAMES)), ("launches", C.c_uint64 * len(K_NAMES))]

    def as_dict(self):
        return {k: (self.total_ms[i], int(self.launches[i])) for i, k in enumerate(K_NAMES)}


def build() -> None:
    """Compile libmetalgym_amd.so for gfx950 with the package Makefile."""
    jobs = str(min(16, os.cpu_count() or 1))
    subprocess.run(["make", "-s", "-j", jobs, "-C", HERE], check=True)


_lib = None


def lib():
    """Load the C ABI library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (no fallback exists)")
    L = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
    I = C.c_int
    sig = {
        "mg_last_error": (C.c_char_p, []),
        "mg_abi_version": (I, []),
        "mg_device_count": (I, [P]),
        "mg_malloc": (I, [P, C.c_size_t]),
        "mg_free": (I, [P]),
        "mg_host_alloc": (I, [P, C.c_size_t]),
        "mg_host_free": (I, [P]),
        "mg_memcpy_h2d": (I, [P, P, C.c_size_t]),
        "mg_memcpy_d2h": (I, [P, P, C.c_size_t]),
        "mg_memcpy_d2d": (I, [P, P, C.c_size_t]),
        "mg_memset": (I, [P, I, C.c_size_t]),
        "mg_synchronize": (I, []),
        "mg_env_register": (I, [P]),
        "mg_env_lookup": (I, [C.c_char_p, P]),
        "mg_env_count": (I, []),
        "mg_env_name": (C.c_char_p, [I]),
        "mg_gym_create": (I, [C.c_char_p, u32, u32, P]),
        "mg_gym_destroy": (I, [P]),
        "mg_gym_buffers_get": (I, [P, P]),
        "mg_gym_step_into": (I, [P, P, P, P]),
        "mg_gym_run": (I, [P]),
        "mg_gym_rollout_random": (I, [P, u32, P, P, P, P]),
        "mg_gym_rollout_given": (I, [P, u32, P, P, P, P]),
        "mg_gym_sync": (I, [P]),
        "mg_ppo_check_config": (I, [C.c_char_p, u32, P]),
        "mg_ppo_create": (I, [P, P, P]),
        "mg_ppo_destroy": (I, [P]),
        "mg_ppo_config_get": (I, [P, P]),
        "mg_ppo_set_hparams": (I, [P, P]),
        "mg_ppo_get_hparams": (I, [P, P]),
        "mg_ppo_collect": (I, [P]),
        "mg_ppo_train": (I, [P, u32]),
        "mg_ppo_train_block": (I, [P, u32]),
        "mg_ppo_forward": (I, [P, P, u32]),
        "mg_ppo_train_block_noalloc": (I, [P, u32, P]),
        "mg_ppo_last_stats": (I, [P, P]),
        "mg_ppo_train_stats": (I, [P, P, u32, P]),
        "mg_ppo_slots_get": (I, [P, P]),
        "mg_ppo_head": (I, [P, P, P, P]),
        "mg_ppo_policy": (I, [P, P]),
        "mg_ppo_set_params": (I, [P, P, u32]),
        "mg_ppo_params_updated": (I, [P]),
        "mg_ppo_adam_state": (I, [P, P, P, P]),
        "mg_ppo_train_capture": (I, [P, u32, P, P, P, P]),
        "mg_ppo_set_log_std": (I, [P, f32]),
        "mg_ppo_last_order": (I, [P, P, u32, P]),
        "mg_ppo_sample": (I, [P, P, u32, P, P, P, P]),
        "mg_gae": (I, [P, P, P, P, P, u32, u32, u32, u32, f32, f32, P, P]),
        "mg_timing_enable": (I, [I]),
        "mg_timing_get": (I, [P]),
        "mg_timing_reset": (I, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        raise CapiError(rc, lib().mg_last_error().decode())


def env_names():
    L = lib()
    return [L.mg_env_name(i).decode() for i in range(L.mg_env_count())]


def env_desc(kernel: str) -> EnvDesc:
    out = C.POINTER(EnvDesc)()
    check(lib().mg_env_lookup(kernel.encode(), C.byref(out)))
    return out.contents


def timing_enable(on: bool = True) -> None:
    check(lib().mg_timing_enable(1 if on else 0))


def timing_reset() -> None:
    check(lib().mg_timing_reset())


def timing_get() -> dict:
    t = KernelTimes()
    check(lib().mg_timing_get(C.byref(t)))
    return t.as_dict()


class DeviceBuffer:
    """A device allocation made through mg_malloc."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().mg_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().mg_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().mg_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def zero(self) -> None:
        check(lib().mg_memset(self.ptr, 0, self.nbytes))

    def free(self) -> None:
        if self.ptr:
            lib().mg_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def d2h(ptr: int, dtype, shape) -> np.ndarray:
    out = np.empty(shape, dtype)
    if out.nbytes:
        check(lib().mg_memcpy_d2h(out.ctypes.data, ptr, out.nbytes))
    return out


def h2d(ptr: int, a: np.ndarray) -> None:
    a = np.ascontiguousarray(a)
    if a.nbytes:
        check(lib().mg_memcpy_h2d(ptr, a.ctypes.data, a.nbytes))


class Gym:
    """mg_gym_* (gym.h:15-122)."""

    def __init__(self, kernel: str, n: int, seed: int = 0):
        self.kernel = kernel
        h = C.c_void_p()
        check(lib().mg_gym_create(kernel.encode(), n, seed, C.byref(h)))
        self.h = h.value
        b = GymBuffers()
        check(lib().mg_gym_buffers_get(self.h, C.byref(b)))
        self.buf = b
        self.n = n
        d = b.env.contents
        self.state_bytes, self.action_bytes = d.state_bytes, d.action_bytes
        self.obs_dim, self.act_dim, self.continuous = d.obs_dim, d.act_dim, bool(d.continuous)
        self.action_dtype = np.float32 if self.continuous else np.int32

    def action_shape(self, *lead):
        return tuple(lead) + ((self.act_dim,) if self.continuous else ())

    def destroy(self) -> None:
        if self.h:
            lib().mg_gym_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def sync(self) -> None:
        check(lib().mg_gym_sync(self.h))

    # host copies of the live buffers
    def state(self) -> np.ndarray:
        self.sync()
        return d2h(self.buf.state, np.uint8, (self.n * self.state_bytes,))

    def rng(self) -> np.ndarray:
        self.sync()
        return d2h(self.buf.rng, np.uint32, (self.n,))

    def done(self) -> np.ndarray:
        self.sync()
        return d2h(self.buf.done, np.uint8, (self.n,))

    def obs(self) -> np.ndarray:
        self.sync()
        return d2h(self.buf.obs, np.float32, (self.n, self.obs_dim))

    def reward(self) -> np.ndarray:
        self.sync()
        return d2h(self.buf.reward, np.float32, (self.n,))

    def set_actions(self, a: np.ndarray) -> None:
        h2d(self.buf.actions, np.ascontiguousarray(a, self.action_dtype))

    def run(self) -> None:
        check(lib().mg_gym_run(self.h))
        self.sync()

    def step_into(self, actions_ptr: int, obs_ptr: int, reward_ptr: int) -> None:
        """gym.h:94-108 (encodeStep): one step reading device actions and writing
        device obs and rewards at the given addresses. Asynchronous."""
        check(lib().mg_gym_step_into(self.h, actions_ptr, obs_ptr, reward_ptr))

    def _slot_bufs(self, steps):
        n = self.n
        acts = DeviceBuffer(steps * n * self.action_bytes)
        obs = DeviceBuffer(steps * n * self.obs_dim * 4)
        rew = DeviceBuffer(steps * n * 4)
        dn = DeviceBuffer(steps * n)
        return acts, obs, rew, dn

    def rollout_random(self, steps: int, bufs=None, sync: bool = True):
        bufs = bufs or self._slot_bufs(steps)
        acts, obs, rew, dn = bufs
        check(lib().mg_gym_rollout_random(self.h, steps, acts.ptr, obs.ptr, rew.ptr, dn.ptr))
        if sync:
            self.sync()
        return bufs

    def rollout_given(self, steps: int, actions: np.ndarray):
        acts_in = DeviceBuffer.from_array(np.ascontiguousarray(actions, self.action_dtype))
        _, obs, rew, dn = self._slot_bufs(steps)
        check(lib().mg_gym_rollout_given(self.h, steps, acts_in.ptr, obs.ptr, rew.ptr, dn.ptr))
        self.sync()
        return acts_in, obs, rew, dn

    def download_slots(self, bufs, steps):
        acts, obs, rew, dn = bufs
        n = self.n
        return (acts.download(self.action_dtype, self.action_shape(steps, n)),
                obs.download(np.float32, (steps, n, self.obs_dim)),
                rew.download(np.float32, (steps, n)), dn.download(np.uint8, (steps, n)))


class PPOModel:
    """mg_ppo_* (model/ppo.h:106-1009)."""

    def __init__(self, gym: Gym, embed=128, scale=4, layers=2, lr=3e-4, horizon=32, seed=0, minibatch=0,
                 precision="fp32"):
        self.gym = gym
        cfg = PPOConfig(embed, scale, layers, horizon, minibatch, seed, lr, {"fp32": 0, "bf16": 1}[precision])
        h = C.c_void_p()
        check(lib().mg_ppo_create(gym.h, C.byref(cfg), C.byref(h)))
        self.h = h.value
        self.cfg = cfg
        self.T = horizon
        self.n = gym.n
        pv = PolicyView()
        check(lib().mg_ppo_policy(self.h, C.byref(pv)))
        self.pv = pv
        s = PPOSlots()
        check(lib().mg_ppo_slots_get(self.h, C.byref(s)))
        self.slots = s

    def policy(self) -> PolicyView:
        """mg_ppo_policy: the device view, its fragment-tiled copies current."""
        pv = PolicyView()
        check(lib().mg_ppo_policy(self.h, C.byref(pv)))
        return pv

    def destroy(self) -> None:
        if self.h:
            lib().mg_ppo_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    @property
    def hparams(self) -> PPOHParams:
        hp = PPOHParams()
        check(lib().mg_ppo_get_hparams(self.h, C.byref(hp)))
        return hp

    @hparams.setter
    def hparams(self, hp: PPOHParams) -> None:
        check(lib().mg_ppo_set_hparams(self.h, C.byref(hp)))

    def collect(self) -> None:
        check(lib().mg_ppo_collect(self.h))

    def train(self, epochs: int = 4) -> None:
        check(lib().mg_ppo_train(self.h, epochs))

    def train_block(self, block: int) -> None:
        check(lib().mg_ppo_train_block(self.h, block))

    def train_block_noalloc(self, block: int, stats_ptr: int = None) -> None:
        """mg_ppo_train_block_noalloc: asynchronous; LossStats to the device
        pointer stats_ptr (6 floats) if given."""
        check(lib().mg_ppo_train_block_noalloc(self.h, block, stats_ptr))

    def forward(self, obs: np.ndarray) -> np.ndarray:
        obs = np.ascontiguousarray(obs, np.float32)
        buf = DeviceBuffer.from_array(obs)
        check(lib().mg_ppo_forward(self.h, buf.ptr, obs.shape[0]))
        return self.head()

    def head(self) -> np.ndarray:
        p, rows, hd = C.c_void_p(), u32(), u32()
        check(lib().mg_ppo_head(self.h, C.byref(p), C.byref(rows), C.byref(hd)))
        return d2h(p.value, np.float32, (rows.value, hd.value))

    def last_stats(self) -> LossStats:
        st = LossStats()
        check(lib().mg_ppo_last_stats(self.h, C.byref(st)))
        return st

    def train_stats(self) -> np.ndarray:
        cnt = u32()
        check(lib().mg_ppo_train_stats(self.h, None, 0, C.byref(cnt)))
        out = (LossStats * max(1, cnt.value))()
        check(lib().mg_ppo_train_stats(self.h, out, cnt.value, C.byref(cnt)))
        return np.array([out[i].as_tuple() for i in range(cnt.value)], np.float32).reshape(-1, 6)

    def last_order(self) -> np.ndarray:
        cnt = u32()
        check(lib().mg_ppo_last_order(self.h, None, 0, C.byref(cnt)))
        out = np.zeros(max(1, cnt.value), np.uint32)
        check(lib().mg_ppo_last_order(self.h, out.ctypes.data, cnt.value, C.byref(cnt)))
        return out[:cnt.value]

    def params(self) -> np.ndarray:
        return d2h(self.pv.params, np.float32, (self.pv.count,))

    def set_params(self, p: np.ndarray) -> None:
        assert p.shape == (self.pv.count,)
        p = np.ascontiguousarray(p, np.float32)
        check(lib().mg_ppo_set_params(self.h, p.ctypes.data_as(C.c_void_p), self.pv.count))

    def adam_state(self):
        m, v, st = C.c_void_p(), C.c_void_p(), u32()
        check(lib().mg_ppo_adam_state(self.h, C.byref(m), C.byref(v), C.byref(st)))
        return d2h(m.value, np.float32, (self.pv.count,)), d2h(v.value, np.float32, (self.pv.count,)), st.value

    def train_capture(self, which: int) -> np.ndarray:
        """Capture `which` (0 LN outputs, 1 relu'd hidden, 2 dh, 3 dV) of the last
        train minibatch as [layers][B][cols]: float32 in fp32 mode; in bf16 mode
        the bfloat16 values unpacked from the row-group-packed layout, as float32."""
        p, rows, cols, layers = C.c_void_p(), u32(), u32(), u32()
        check(lib().mg_ppo_train_capture(self.h, which, C.byref(p), C.byref(rows), C.byref(cols), C.byref(layers)))
        Lr, B, Cc = layers.value, rows.value, cols.value
        if self.pv.precision == 0:
            return d2h(p.value, np.float32, (Lr, B, Cc))
        raw = d2h(p.value, np.uint16, (Lr, B // 8, Cc, 8))
        return (raw.astype(np.uint32) << 16).view(np.float32).transpose(0, 1, 3, 2).reshape(Lr, B, Cc)

    def set_log_std(self, value: float) -> None:
        check(lib().mg_ppo_set_log_std(self.h, value))

    def download_slots(self) -> dict:
        s, n, T, g = self.slots, self.n, self.T, self.gym
        return {
            "obs": d2h(s.obs, np.float32, (T + 1, n, g.obs_dim)),
            "actions": d2h(s.actions, g.action_dtype, g.action_shape(T, n)),
            "logp": d2h(s.logp, np.float32, (T, n)),
            "value": d2h(s.value, np.float32, (T, n)),
            "reward": d2h(s.reward, np.float32, (T, n)),
            "done": d2h(s.done, np.uint8, (T, n)),
            "adv": d2h(s.advantage, np.float32, (T, n)),
            "ret": d2h(s.ret, np.float32, (T, n)),
        }

    def upload_slots(self, d: dict) -> None:
        s, g = self.slots, self.gym
        for key, ptr, dt in (("obs", s.obs, np.float32), ("actions", s.actions, g.action_dtype),
                             ("logp", s.logp, np.float32), ("value", s.value, np.float32),
                             ("reward", s.reward, np.float32), ("done", s.done, np.uint8),
                             ("adv", s.advantage, np.float32), ("ret", s.ret, np.float32)):
            if key in d:
                h2d(ptr, np.ascontiguousarray(d[key], dt))

    def sample(self, head: np.ndarray, rng: np.ndarray):
        rows = head.shape[0]
        hb = DeviceBuffer.from_array(np.ascontiguousarray(head, np.float32))
        rb = DeviceBuffer.from_array(np.ascontiguousarray(rng, np.uint32))
        g = self.gym
        ab = DeviceBuffer(rows * g.action_bytes)
        lb = DeviceBuffer(rows * 4)
        vb = DeviceBuffer(rows * 4)
        check(lib().mg_ppo_sample(self.h, hb.ptr, rows, rb.ptr, ab.ptr, lb.ptr, vb.ptr))
        return (ab.download(g.action_dtype, g.action_shape(rows)), lb.download(np.float32, (rows,)),
                vb.download(np.float32, (rows,)), rb.download(np.uint32, (rows,)))
