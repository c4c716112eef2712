"""Benchmark of the rollout-and-policy hot path on one MI355X.

Headline: CartPole with policy, collect() at 262144 envs, T = 32, the 2-block
residual MLP (embed 128, hidden 512) -- the reference's collect benchmark at its largest
size. One step = one collect() (262144 x 32 env steps, policy forward on fp32
MFMA, sampling, env step, GAE). Inputs are synthetic (seeded envs and weights)
and resident on the GPU. The other configurations (random policy, full PPO loop,
continuous, VoxelNav16) are reported as extra fields of the same JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA = 157.3e12  # FLOP/s, MI355X dense fp32 matrix
PEAK_HBM = 8.0e12          # B/s
E, H, L = 128, 512, 2


def fwd_flop(O, A, layers=L, hidden=H):
    """Algorithmic FLOP of one policy forward row (embed, blocks, head)."""
    return 2 * (O * E + 2 * layers * E * hidden + E * (A + 1))


def bwd_flop(O, A, layers=L, hidden=H):
    """dX chain + weight gradients of one row (no dX for the embed)."""
    dx = 2 * (2 * layers * E * hidden + E * (A + 1))
    dw = fwd_flop(O, A, layers, hidden)
    return dx + dw


def sync():
    import metalgym_amd as mg

    mg.lib().mg_synchronize()


def kernel_avg_ms(times, k):
    tot, cnt = times[k]
    return tot / cnt if cnt else float("nan")


def bench_collect(kernel, n, T, steps, warmup, O, A, precision="fp32", layers=L):
    import metalgym_amd as mg

    gym = mg.Gym(kernel, n, 0)
    model = mg.PPOModel(gym, horizon=T, precision=precision, layers=layers)
    for _ in range(warmup):
        model.collect()
    sync()
    mg.timing_reset()
    mg.timing_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        model.collect()
    sync()
    dt = time.perf_counter() - t0
    mg.timing_enable(False)
    times = mg.timing_get()
    return gym, model, dt, times


# Envs whose steps write only a leading header of State (STEP_WRITES in the
# env's header, in bytes here): the split rollout writes the rest of an env's
# state back only if the env reset during the launch.
STEP_WRITE_BYTES = {"rollout_voxelnav16": 32}


def rollout_bytes(gym, n, T, resets=None):
    """HBM bytes of one random rollout launch that no layout avoids: the T
    slots (obs, action, reward, done), each env's rng and done read and written
    once, and its state read once and written back once: whole, or for an env
    of STEP_WRITE_BYTES its header plus, for each of the `resets` envs that
    reset in the launch, the rest. CartPole: 26.5 B per env-step. VoxelNav16:
    129 B of slots per env-step, its 4128-byte state read once per launch."""
    slot = 4 * gym.obs_dim + gym.action_bytes + 4 + 1
    hdr = STEP_WRITE_BYTES.get(gym.kernel)
    if hdr is None or resets is None:
        return n * T * slot + n * 2 * (gym.state_bytes + 4 + 1)
    return n * T * slot + n * 2 * (4 + 1) + n * (gym.state_bytes + hdr) + resets * (gym.state_bytes - hdr)


def bench_random(n, T, reps, kernel="rollout_cartpole", hbm=True):
    """Random-policy rollouts, with the launch's unavoidable HBM bytes
    (rollout_bytes) over the kernel's event-timed duration."""
    import numpy as np
    import metalgym_amd as mg

    gym = mg.Gym(kernel, n, 0)
    bufs = gym.rollout_random(T)
    sync()
    # an env of STEP_WRITE_BYTES writes its whole state back only in a launch
    # in which it resets, which it does iff its done flag was set at the end
    # of the previous launch or at any step of this one but the last: each
    # launch's done slots are read back after it (outside the timed sum)
    partial = hbm and kernel in STEP_WRITE_BYTES
    resets = 0
    if partial:
        dn = bufs[3]
        prev = dn.download(np.uint8, (T, n))[T - 1].astype(bool)
    mg.timing_reset()
    mg.timing_enable(True)
    if partial:
        dt = 0.0
        for _ in range(reps):
            t0 = time.perf_counter()
            gym.rollout_random(T, bufs, sync=False)
            sync()
            dt += time.perf_counter() - t0
            d = dn.download(np.uint8, (T, n)).astype(bool)
            resets += int((prev | d[:T - 1].any(axis=0)).sum())
            prev = d[T - 1]
    else:
        t0 = time.perf_counter()
        for _ in range(reps):
            gym.rollout_random(T, bufs, sync=False)
        sync()
        dt = time.perf_counter() - t0
    mg.timing_enable(False)
    times = mg.timing_get()
    kms = kernel_avg_ms(times, "rollout")
    out = {"env_steps_per_s": reps * n * T / dt, "kernel_us": kms * 1e3}
    if hbm:
        bytes_launch = rollout_bytes(gym, n, T, resets / reps if partial else None)
        if partial:
            out["resets_per_launch"] = resets / reps
        out["bytes_per_launch"] = bytes_launch
        out["hbm_GBps"] = bytes_launch / (kms * 1e-3) / 1e9
        out["hbm_frac"] = bytes_launch / (kms * 1e-3) / PEAK_HBM
    return out


def copy_floor_us(nbytes, reps=20):
    """Device-to-device copies moving nbytes of HBM traffic (nbytes / 2 read,
    nbytes / 2 written), each between regions no earlier copy touched, timed
    with HIP events by the library (mg_memcpy_d2d); the median in us. The size
    floor of a kernel with that much traffic (Adam's 28 B per parameter)."""
    import metalgym_amd as mg

    half = (nbytes // 2 + 255) // 256 * 256
    src, dst = mg.DeviceBuffer(reps * half), mg.DeviceBuffer(reps * half)
    src.zero()
    dst.zero()
    times = []
    for k in range(reps):
        mg.timing_reset()
        mg.timing_enable(True)
        mg.lib().mg_memcpy_d2d(dst.ptr + k * half, src.ptr + k * half, half)
        mg.timing_enable(False)
        tot, cnt = mg.timing_get()["copy"]
        times.append(tot / cnt * 1e3)
    times.sort()
    return times[len(times) // 2]


def bench_full(kernel, n, T, iters, O, A, epochs=4, precision="fp32", layers=L, floor=False):
    """The full loop (collect + train(epochs)), iters iterations untimed by
    events, then one iteration with per-kernel HIP events. floor: also time a
    device copy of Adam's byte count (copy_floor_us) in the same process."""
    import metalgym_amd as mg

    gym = mg.Gym(kernel, n, 0)
    model = mg.PPOModel(gym, horizon=T, precision=precision, layers=layers)
    model.collect()
    model.train(1)
    sync()
    # throughput untimed (per-kernel events would add their own gaps), then one
    # iteration with per-kernel events for the breakdown
    t0 = time.perf_counter()
    for _ in range(iters):
        model.collect()
        model.train(epochs)
    sync()
    dt = time.perf_counter() - t0
    st = model.last_stats()
    mg.timing_reset()
    mg.timing_enable(True)
    model.collect()
    model.train(epochs)
    sync()
    mg.timing_enable(False)
    times = mg.timing_get()
    B = min(n, 4096)
    out = {"env_steps_per_s": iters * n * T / dt, "s_per_iter": dt / iters,
           "minibatches_per_iter": epochs * T * n // B,
           "last_stats": dict(zip(["policy", "value", "entropy", "approx_kl", "clip_frac", "grad_norm"],
                                  [round(x, 6) for x in st.as_tuple()]))}
    kern = {}
    for k in ("collect", "gae", "adv_stats", "train_rows", "train_dw", "grad_reduce", "adam"):
        if times[k][1]:  # at the default shape grad_reduce is fused into train_dw
            kern[k + "_us"] = round(kernel_avg_ms(times, k) * 1e3, 2)
    tr = kernel_avg_ms(times, "train_rows") * 1e-3
    dw = kernel_avg_ms(times, "train_dw") * 1e-3
    ad = kernel_avg_ms(times, "adam") * 1e-3
    count = model.pv.count
    fw, bw = fwd_flop(O, A, layers), bwd_flop(O, A, layers)
    kern["train_rows_TFLOPs"] = round(B * (fw + bw - fw) / tr / 1e12, 2)
    kern["train_dw_TFLOPs"] = round(B * fw / dw / 1e12, 2)
    kern["adam_GBps"] = round(count * 28 / ad / 1e9, 1)
    if floor:
        fl = copy_floor_us(count * 28)
        kern["adam_copy_floor_us"] = round(fl, 2)
        kern["adam_over_copy_floor"] = round(ad * 1e6 / fl, 2)
    out["kernels"] = kern
    return out


def host_cores():
    """The host's logical CPUs, and those this process may run on."""
    cores = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = cores
    return cores, usable


def cpu_threads():
    """Oracle threads: the usable host CPUs, at most 16 (a GPU box's CPU share)."""
    return max(1, min(16, host_cores()[1]))


def cpu_baseline(target_s=10.0):
    """The CPU oracle's collect() on a bounded slice of the headline workload
    (CartPole, T = 32, same network), on the host's cores."""
    import oracle as orc

    threads = cpu_threads()
    T = 32
    d = orc.dims(orc.CARTPOLE)
    params = orc.init_params(d, 0)

    def run(n):
        g = orc.GymState(orc.CARTPOLE, n, 0)
        s = orc.Slots(orc.CARTPOLE, n, T)
        t0 = time.perf_counter()
        orc.collect(g, d, params, T, s, first=True, threads=threads)
        return time.perf_counter() - t0

    n = 64 * threads
    dt = run(n)
    n = int(max(64, min(262144, n * target_s / max(dt, 1e-3))) // 64 * 64)
    dt = run(n)
    cores, usable = host_cores()
    return {"value": n * T / dt, "unit": "env steps/s", "cores": threads, "kind": "port",
            "host_cores": cores, "usable_cores": usable,
            "sample": f"oracle collect() of {n} of the 262144 CartPole envs, T=32, 2-block MLP, fp32, "
                      f"{threads} threads, {dt:.1f} s"}


def cpu_extras(threads=None):
    """The oracle on the host for every benchmark configuration, each bounded to
    a few seconds and labelled with its scope (T = 32, the 2-block MLP, 4096-row
    minibatches, 4 epochs; an iteration is one collect of all n envs plus
    4 n T / 4096 minibatches):
      config 1  random rollouts of 4096 and 262144 CartPole envs (whole launches);
      config 2  collect() of 4096 CartPole envs (whole; 262144 is the headline
                cpu_baseline's slice);
      config 3  the full loop at 4096 envs (one whole collect, a few timed
                minibatches) and at 262144 envs (scoped: a collect of a slice
                of the envs and a few timed minibatches, combined at the
                measured per-env-step and per-minibatch costs);
      config 4  CartPoleContinuous full loop at 65536 and 262144 envs (scoped
                the same way, one measurement for both sizes);
      config 5  VoxelNav16 collect and full loop at 262144 envs (scoped).
    Every entry states its threads, the host's cores and its scope."""
    import numpy as np

    import oracle as orc

    threads = threads or cpu_threads()
    cores, usable = host_cores()
    T, B, epochs = 32, 4096, 4
    out = {}

    def repeated(fn, min_s=2.0):
        """Calls fn until min_s seconds have passed; returns (calls, seconds)."""
        calls, t0 = 0, time.perf_counter()
        while True:
            fn(calls)
            calls += 1
            dt = time.perf_counter() - t0
            if dt >= min_s:
                return calls, dt

    def entry(value, scope, **kw):
        e = {"env_steps_per_s": value, "cores": threads, "threads": threads, "host_cores": cores,
             "usable_cores": usable, "kind": "port", "scope": scope}
        e.update(kw)
        return e

    for n in (4096, 262144):  # config 1
        g = orc.GymState(orc.CARTPOLE, n, 0)
        reps, dt = repeated(lambda _: orc.rollout(g, T, random=True, threads=threads))
        out[f"cpu_random_{n}"] = entry(reps * n * T / dt, f"{reps} whole random rollouts of {n} CartPole envs x 32 "
                                                          f"in {dt:.1f} s")

    def collect_and_minibatches(env, n_collect, min_mb):
        """Collect of n_collect envs (repeated for 2 s) and min_mb timed
        minibatches of B rows of its slots; returns seconds per env-step of
        collect, seconds per minibatch and the counts."""
        d = orc.dims(env)
        params = orc.init_params(d, 0)
        g = orc.GymState(env, n_collect, 0)
        slots = orc.Slots(env, n_collect, T)
        nc, dc = repeated(lambda c: orc.collect(g, d, params, T, slots, first=(c == 0), threads=threads))
        hp = orc.hparams()
        P, M, V = params.copy(), np.zeros_like(params), np.zeros_like(params)

        def minibatch(c):
            t = c % T
            rows = slice(0, B)
            orc.train_minibatch(d, hp, P, M, V, c + 1, slots.obs[t, rows], slots.actions[t, rows],
                                slots.adv[t, rows], slots.ret[t, rows], slots.logp[t, rows], threads=threads)

        t0 = time.perf_counter()
        for c in range(min_mb):
            minibatch(c)
        dm = time.perf_counter() - t0
        return dc / (nc * n_collect * T), dm / min_mb, nc, min_mb

    # config 2 at 4096 and config 3 at 4096: whole collects, timed minibatches
    sc, sm, nc, k = collect_and_minibatches(orc.CARTPOLE, 4096, 4)
    out["cpu_collect_4096"] = entry(1.0 / sc, f"{nc} whole collects of 4096 CartPole envs x 32")
    it = 4096 * T * sc + epochs * (4096 * T // B) * sm
    out["cpu_full_ppo_4096"] = entry(4096 * T / it, f"{nc} whole collects of 4096 envs x 32 and {k} minibatches of "
                                                    f"4096 rows ({sm:.2f} s each); iteration = collect + 128 "
                                                    f"minibatches", s_per_minibatch=sm)
    # the 262144-env loops, scoped: a 16384-env collect slice and a few minibatches
    for key, env, sizes in (("cpu_full_ppo", orc.CARTPOLE, (262144,)),
                            ("cpu_continuous_full_ppo", orc.CARTPOLE_CONT, (65536, 262144)),
                            ("cpu_voxelnav16_full_ppo", orc.VOXELNAV16, (262144,))):
        sc, sm, nc, k = collect_and_minibatches(env, 16384, 3)
        for n in sizes:
            mbs = epochs * (n * T // B)
            it = n * T * sc + mbs * sm
            out[f"{key}_{n}"] = entry(n * T / it, f"scoped: {nc} collects of 16384 of the {n} envs x 32 "
                                                  f"({sc * 1e9:.0f} ns per env-step) and {k} minibatches of 4096 rows "
                                                  f"({sm:.2f} s each); iteration = {n} x 32 env-steps of collect + "
                                                  f"{mbs} minibatches at those costs",
                                      s_per_minibatch=sm, collect_env_steps_per_s=1.0 / sc)
        if env == orc.VOXELNAV16:
            out["cpu_voxelnav16_collect_262144"] = entry(1.0 / sc, f"scoped: {nc} collects of 16384 of the 262144 "
                                                                   f"VoxelNav16 envs x 32")
    return out


def pmc_traffic():
    """HBM bytes per collect launch from the committed rocprofv3 --pmc summary, if any."""
    p = os.path.join(ROOT, "profiles", "collect_cartpole_262144_pmc.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def profile_pass(which):
    """Short runs of each kernel for rocprofv3 (--kernel-trace / --pmc): the
    262144-env collect and random rollout, 64 train minibatches, the 4096-env
    collect ("all"; its 16-row tiles), and one 1 GiB
    device-to-device copy whose FETCH_SIZE / WRITE_SIZE calibrate the counters
    ("all" adds 64 copies of the Adam step's byte count, its size floor).
    "bf16": the collect and the minibatches in bf16 mode, and the copy.
    "train": one collect and two train(1) epochs of the 262144-env fp32 loop
    (2048 minibatches each, enqueued back to back as in the benchmark).
    "cfg45": configs 4 and 5 at 262144 envs: three collects and 64 minibatches
    each of CartPoleContinuous and VoxelNav16, eleven VoxelNav16 random rollouts
    (their resets per launch printed), and the 1 GiB copy."""
    import metalgym_amd as mg

    n, T = 262144, 32
    if which == "cfg45":  # configs 4 and 5: the continuous and VoxelNav16 kernels
        for kernel in ("rollout_cartpole_continuous", "rollout_voxelnav16"):
            gym = mg.Gym(kernel, n, 0)
            model = mg.PPOModel(gym, horizon=T)
            for _ in range(3):
                model.collect()
            sync()
            print(f"profile: 3 collects of {kernel} at 262144 x 32", flush=True)
            for b in range(64):
                mg.lib().mg_ppo_train_block(model.h, b)
            sync()
            print(f"profile: 64 train minibatches of 4096 rows of {kernel}", flush=True)
            del model, gym
        # the bench's launches (one after the gym's first, which resets every
        # env, then ten), each env that resets in a launch counted from the done
        # slots: such an env writes its whole 4128-byte state back
        import numpy as np
        gym = mg.Gym("rollout_voxelnav16", n, 0)
        bufs = gym.rollout_random(T)
        prev = bufs[3].download(np.uint8, (T, n))[T - 1].astype(bool)
        resets = [n]
        for _ in range(10):
            gym.rollout_random(T, bufs)
            d = bufs[3].download(np.uint8, (T, n)).astype(bool)
            resets.append(int((prev | d[:T - 1].any(axis=0)).sum()))
            prev = d[T - 1]
        print(f"profile: 11 random rollouts of rollout_voxelnav16 at 262144 x 32, resets {resets}", flush=True)
        del gym, bufs
        nbytes = 1 << 30
        a, b = mg.DeviceBuffer(nbytes), mg.DeviceBuffer(nbytes)
        a.zero()
        mg.lib().mg_memcpy_d2d(b.ptr, a.ptr, nbytes)
        sync()
        print(f"profile: one device copy of {nbytes} bytes", flush=True)
        return
    if which == "train":
        gym = mg.Gym("rollout_cartpole", n, 0)
        model = mg.PPOModel(gym, horizon=T)
        model.collect()
        for e in range(2):
            model.train(1)
            print(f"profile: train(1) epoch {e} of 2048 minibatches of 4096 rows", flush=True)
        return
    if which in ("collect", "all", "bf16"):
        precision = "bf16" if which == "bf16" else "fp32"
        gym = mg.Gym("rollout_cartpole", n, 0)
        model = mg.PPOModel(gym, horizon=T, precision=precision)
        for _ in range(3):
            model.collect()
        print(f"profile: 3 {precision} collects of 262144 x 32", flush=True)
        if which in ("all", "bf16"):
            for b in range(64):
                mg.lib().mg_ppo_train_block(model.h, b)
            sync()
            print(f"profile: 64 {precision} train minibatches of 4096 rows", flush=True)
        del model, gym
        if which == "all":  # 16-row tiles (the split forward)
            gym = mg.Gym("rollout_cartpole", 4096, 0)
            model = mg.PPOModel(gym, horizon=T)
            for _ in range(3):
                model.collect()
            sync()
            print("profile: 3 fp32 collects of 4096 x 32", flush=True)
            del model, gym
    if which in ("random", "all"):
        gym = mg.Gym("rollout_cartpole", n, 0)
        bufs = gym.rollout_random(T)
        for _ in range(5):
            gym.rollout_random(T, bufs, sync=False)
        sync()
        print("profile: 6 random rollouts of 262144 x 32", flush=True)
        del gym, bufs
    if which in ("copy", "all", "bf16"):
        nbytes = 1 << 30
        a, b = mg.DeviceBuffer(nbytes), mg.DeviceBuffer(nbytes)
        a.zero()
        mg.lib().mg_memcpy_d2d(b.ptr, a.ptr, nbytes)
        sync()
        print(f"profile: one device copy of {nbytes} bytes", flush=True)
        if which == "all":
            # the floor of a kernel of the Adam step's size: copies that move its
            # 28 B per parameter (14 B read + 14 B written), each from and to a
            # region no earlier copy touched (not in L2)
            gym = mg.Gym("rollout_cartpole", 4096, 0)
            small = mg.PPOModel(gym, horizon=T).pv.count * 14
            for k in range(64):
                mg.lib().mg_memcpy_d2d(b.ptr + k * small, a.ptr + k * small, small)
            sync()
            print(f"profile: 64 device copies of {small} bytes", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--profile", choices=["collect", "random", "copy", "all", "bf16", "train", "cfg45"], default=None,
                    help="run short kernel passes for rocprofv3 instead of the benchmark")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X; this build has no multi-GPU path (--gpus must be 1)", file=sys.stderr)
        sys.exit(2)

    import metalgym_amd as mg

    if args.profile:
        profile_pass(args.profile)
        return

    n, T = 262144, 32
    O, A = 4, 2
    gym, model, dt, times = bench_collect("rollout_cartpole", n, T, args.steps, args.warmup, O, A)
    value = args.steps * n * T / dt
    kms = kernel_avg_ms(times, "collect")
    flop_launch = (T + 1) * n * fwd_flop(O, A)
    achieved = flop_launch / (kms * 1e-3)
    gae_ms = kernel_avg_ms(times, "gae")
    line = {
        "metric": "CartPole env steps/s: random, w/ policy, full PPO loop @4096 & 262144 envs",
        "value": value,
        "unit": "env steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded envs and weights)",
        "config": {"workload": "cartpole_collect_with_policy", "envs": n, "horizon": T, "embed": E, "hidden": H,
                   "layers": L, "head": "softmax(2)+value", "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "kernel": "collect_kernel<CartPole,64,false,false>", "achieved": achieved / 1e12,
                     "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s", "frac": achieved / PEAK_FP32_MFMA,
                     "traffic": pmc_traffic(),
                     "traffic_source": "profiles/collect_cartpole_262144_pmc.json: rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE of this kernel (a committed profile, not measured in this run)",
                     "flop_per_launch": flop_launch, "kernel_ms": kms},
        "gae": {"kernel_us": gae_ms * 1e3, "hbm_GBps": (n * T * 17 + n * 4) / (gae_ms * 1e-3) / 1e9},
    }
    del model, gym
    if not args.no_extra:
        extra = {}
        extra["random_4096"] = bench_random(4096, 32, 50)
        extra["random_262144"] = bench_random(262144, 32, 20)
        _, _, dt4, t4 = bench_collect("rollout_cartpole", 4096, 32, 20, 2, O, A)
        extra["collect_4096"] = {"env_steps_per_s": 20 * 4096 * 32 / dt4,
                                 "vs_published_m4_3.8M": 20 * 4096 * 32 / dt4 / 3.8e6}
        extra["full_ppo_4096"] = bench_full("rollout_cartpole", 4096, 32, 5, O, A)
        extra["full_ppo_4096"]["vs_published_m4_296K"] = extra["full_ppo_4096"]["env_steps_per_s"] / 296e3
        extra["full_ppo_262144"] = bench_full("rollout_cartpole", 262144, 32, 1, O, A, floor=True)
        # the README's 1-block rows (published Apple M4 figures: 6.7 M collect, 496 K full loop)
        _, _, dt1, _ = bench_collect("rollout_cartpole", 4096, 32, 20, 2, O, A, layers=1)
        extra["collect_4096_1block"] = {"env_steps_per_s": 20 * 4096 * 32 / dt1,
                                        "vs_published_m4_6.7M": 20 * 4096 * 32 / dt1 / 6.7e6}
        extra["full_ppo_4096_1block"] = bench_full("rollout_cartpole", 4096, 32, 5, O, A, layers=1)
        extra["full_ppo_4096_1block"]["vs_published_m4_496K"] = \
            extra["full_ppo_4096_1block"]["env_steps_per_s"] / 496e3
        _, _, dtc, tc = bench_collect("rollout_cartpole_continuous", 262144, 32, 3, 1, 4, 1)
        kc = kernel_avg_ms(tc, "collect")
        extra["continuous_collect_262144"] = {"env_steps_per_s": 3 * 262144 * 32 / dtc, "collect_ms": kc,
                                              "mfma_frac": 33 * 262144 * fwd_flop(4, 1) / (kc * 1e-3) / PEAK_FP32_MFMA}
        extra["continuous_full_ppo_65536"] = bench_full("rollout_cartpole_continuous", 65536, 32, 2, 4, 1)
        extra["continuous_full_ppo_262144"] = bench_full("rollout_cartpole_continuous", 262144, 32, 1, 4, 1)
        _, _, dtv, tv = bench_collect("rollout_voxelnav16", 262144, 32, 3, 1, 30, 6)
        kv = kernel_avg_ms(tv, "collect")
        extra["voxelnav16_collect_262144"] = {"env_steps_per_s": 3 * 262144 * 32 / dtv, "collect_ms": kv,
                                              "mfma_frac": 33 * 262144 * fwd_flop(30, 6) / (kv * 1e-3) / PEAK_FP32_MFMA}
        extra["voxelnav16_random_262144"] = bench_random(262144, 32, 10, "rollout_voxelnav16")
        extra["voxelnav16_full_ppo_262144"] = bench_full("rollout_voxelnav16", 262144, 32, 1, 30, 6)
        # the reference's heightmap VoxelNav at its README configuration (4096 envs,
        # 2-block policy; published Apple M4 figures: 7.9 M, 2.4 M, 265 K)
        vr = bench_random(4096, 32, 20, "rollout_voxelnav", hbm=False)
        vr["vs_published_m4_7.9M"] = vr["env_steps_per_s"] / 7.9e6
        extra["voxelnav_random_4096"] = vr
        _, _, dtr, _ = bench_collect("rollout_voxelnav", 4096, 32, 10, 2, 40, 6)
        extra["voxelnav_collect_4096"] = {"env_steps_per_s": 10 * 4096 * 32 / dtr,
                                          "vs_published_m4_2.4M": 10 * 4096 * 32 / dtr / 2.4e6}
        extra["voxelnav_full_ppo_4096"] = bench_full("rollout_voxelnav", 4096, 32, 3, 40, 6)
        extra["voxelnav_full_ppo_4096"]["vs_published_m4_265K"] = \
            extra["voxelnav_full_ppo_4096"]["env_steps_per_s"] / 265e3
        extra["voxelnav_random_262144"] = bench_random(262144, 32, 5, "rollout_voxelnav", hbm=False)
        _, _, dtr2, _ = bench_collect("rollout_voxelnav", 262144, 32, 3, 1, 40, 6)
        extra["voxelnav_collect_262144"] = {"env_steps_per_s": 3 * 262144 * 32 / dtr2}
        # bf16 matrix operands (the reference's matmul precision), policy forward only
        _, _, dtb, tb = bench_collect("rollout_cartpole", 262144, 32, 5, 2, O, A, precision="bf16")
        kb = kernel_avg_ms(tb, "collect")
        extra["bf16_collect_262144"] = {"env_steps_per_s": 5 * 262144 * 32 / dtb, "collect_ms": kb,
                                        "matmul_TFLOPs": flop_launch / (kb * 1e-3) / 1e12}
        _, _, dtb4, _ = bench_collect("rollout_cartpole", 4096, 32, 20, 2, O, A, precision="bf16")
        extra["bf16_collect_4096"] = {"env_steps_per_s": 20 * 4096 * 32 / dtb4,
                                      "vs_published_m4_3.8M": 20 * 4096 * 32 / dtb4 / 3.8e6}
        extra["bf16_full_ppo_262144"] = bench_full("rollout_cartpole", 262144, 32, 1, O, A, precision="bf16")
        extra["bf16_full_ppo_4096"] = bench_full("rollout_cartpole", 4096, 32, 5, O, A, precision="bf16")
        extra["bf16_full_ppo_4096"]["vs_published_m4_296K"] = extra["bf16_full_ppo_4096"]["env_steps_per_s"] / 296e3
        line["extra"] = extra
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
        if "extra" in line:
            line["extra"].update(cpu_extras())
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
