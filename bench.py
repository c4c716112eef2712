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


def bench_random(n, T, reps, kernel="rollout_cartpole", hbm=True):
    """Random-policy rollouts; the HBM figures are CartPole's slot and state
    bytes (26.5 B per env-step)."""
    import metalgym_amd as mg

    gym = mg.Gym(kernel, n, 0)
    bufs = gym.rollout_random(T)
    sync()
    mg.timing_reset()
    mg.timing_enable(True)
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
        bytes_launch = n * T * 25 + n * 2 * (20 + 4 + 1)
        out["hbm_GBps"] = bytes_launch / (kms * 1e-3) / 1e9
        out["hbm_frac"] = bytes_launch / (kms * 1e-3) / PEAK_HBM
    return out


def bench_full(kernel, n, T, iters, O, A, epochs=4, precision="fp32", layers=L):
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
    out["kernels"] = kern
    return out


def cpu_baseline(target_s=10.0):
    """The CPU oracle's collect() on a bounded slice of the headline workload
    (CartPole, T = 32, same network), on the host's cores."""
    import numpy as np

    import oracle as orc

    threads = max(1, min(16, os.cpu_count() or 1))
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
    return {"value": n * T / dt, "unit": "env steps/s", "cores": threads, "kind": "port",
            "sample": f"oracle collect() of {n} of the 262144 CartPole envs, T=32, 2-block MLP, fp32, "
                      f"{threads} threads, {dt:.1f} s"}


def cpu_extras(threads=None):
    """The oracle on the host for the other benchmark configurations, bounded:
    the random rollout at 262144 envs (config 1), and the full PPO loop at 4096
    envs (config 3) from one collect and a few timed minibatches, an iteration
    being one collect plus 4 epochs x 32 minibatches of 4096 rows."""
    import numpy as np

    import oracle as orc

    threads = threads or max(1, min(16, os.cpu_count() or 1))
    T = 32
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

    n = 262144
    g = orc.GymState(orc.CARTPOLE, n, 0)
    reps, dt = repeated(lambda _: orc.rollout(g, T, random=True, threads=threads))
    out["cpu_random_262144"] = {"env_steps_per_s": reps * n * T / dt, "cores": threads, "kind": "port",
                                "sample": f"oracle random rollouts of 262144 CartPole envs x 32, {reps} in {dt:.1f} s"}
    n = 4096
    d = orc.dims(orc.CARTPOLE)
    params = orc.init_params(d, 0)
    g = orc.GymState(orc.CARTPOLE, n, 0)
    slots = orc.Slots(orc.CARTPOLE, n, T)
    nc, dc = repeated(lambda c: orc.collect(g, d, params, T, slots, first=(c == 0), threads=threads))
    tc = dc / nc
    hp = orc.hparams()
    P, M, V = params.copy(), np.zeros_like(params), np.zeros_like(params)

    def minibatch(c):
        t = c % T
        orc.train_minibatch(d, hp, P, M, V, c + 1, slots.obs[t], slots.actions[t], slots.adv[t], slots.ret[t],
                            slots.logp[t], threads=threads)

    k, dm = repeated(minibatch)
    tm = dm / k
    it = tc + 4 * T * tm
    out["cpu_full_ppo_4096"] = {"env_steps_per_s": n * T / it, "cores": threads, "kind": "port",
                                "sample": f"oracle collect of 4096 envs x 32 ({nc} in {dc:.1f} s) and {k} minibatches "
                                          f"of 4096 rows ({tm:.2f} s each); iteration = collect + 128 minibatches"}
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
    (2048 minibatches each, enqueued back to back as in the benchmark)."""
    import metalgym_amd as mg

    n, T = 262144, 32
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
    ap.add_argument("--profile", choices=["collect", "random", "copy", "all", "bf16", "train"], default=None,
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
                     "traffic": pmc_traffic(), "flop_per_launch": flop_launch, "kernel_ms": kms},
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
        extra["full_ppo_262144"] = bench_full("rollout_cartpole", 262144, 32, 1, O, A)
        # the README's 1-block rows (published Apple M4 figures: 6.7 M collect, 496 K full loop)
        _, _, dt1, _ = bench_collect("rollout_cartpole", 4096, 32, 20, 2, O, A, layers=1)
        extra["collect_4096_1block"] = {"env_steps_per_s": 20 * 4096 * 32 / dt1,
                                        "vs_published_m4_6.7M": 20 * 4096 * 32 / dt1 / 6.7e6}
        extra["full_ppo_4096_1block"] = bench_full("rollout_cartpole", 4096, 32, 5, O, A, layers=1)
        extra["full_ppo_4096_1block"]["vs_published_m4_496K"] = \
            extra["full_ppo_4096_1block"]["env_steps_per_s"] / 496e3
        _, _, dtc, _ = bench_collect("rollout_cartpole_continuous", 262144, 32, 3, 1, 4, 1)
        extra["continuous_collect_262144"] = {"env_steps_per_s": 3 * 262144 * 32 / dtc}
        extra["continuous_full_ppo_65536"] = bench_full("rollout_cartpole_continuous", 65536, 32, 2, 4, 1)
        extra["continuous_full_ppo_262144"] = bench_full("rollout_cartpole_continuous", 262144, 32, 1, 4, 1)
        _, _, dtv, tv = bench_collect("rollout_voxelnav16", 262144, 32, 3, 1, 30, 6)
        extra["voxelnav16_collect_262144"] = {"env_steps_per_s": 3 * 262144 * 32 / dtv,
                                              "collect_ms": kernel_avg_ms(tv, "collect")}
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
