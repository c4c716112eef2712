// Throughput bench in the shape of the reference's bench/metalrl_bench.cpp:
// argv N and L; warm-up; env-only gym.run() loop; ITERS x (collect, train).
#include <chrono>
#include <cstdio>
#include <cstdlib>

#include "mg/envs/cartpole.h"
#include "mg/ppo.h"

using clk = std::chrono::steady_clock;
static double sec(clk::time_point a, clk::time_point b) { return std::chrono::duration<double>(b - a).count(); }

int main(int argc, char** argv) {
    const uint32_t N = argc > 1 ? std::atoi(argv[1]) : 4096, T = 32;
    const int L = argc > 2 ? std::atoi(argv[2]) : 2;
    const int ITERS = argc > 3 ? std::atoi(argv[3]) : 20;
    Gym<CartPole> gym(N);
    PPOModel<CartPole> model(gym, 128, 4, L, 3e-4f, T);
    std::vector<float> reward(N);
    model.collect();
    model.train();
    auto t0 = clk::now();
    for (int i = 0; i < 1000; i++) gym.run(reward);
    double envOnly = sec(t0, clk::now());
    double collectT = 0, trainT = 0;
    for (int it = 0; it < ITERS; it++) {
        auto a = clk::now();
        model.collect();
        auto b = clk::now();
        model.train();
        auto c = clk::now();
        collectT += sec(a, b);
        trainT += sec(b, c);
    }
    double steps = (double)ITERS * N * T;
    std::printf("N=%u T=%u layers=%d\n", N, T, L);
    std::printf("env step only (gym.run loop):      %10.0f steps/s\n", 1000.0 * N / envOnly);
    std::printf("collect (policy + env + GAE):      %10.0f steps/s\n", steps / collectT);
    std::printf("collect + train (4 epochs):        %10.0f steps/s\n", steps / (collectT + trainT));
    std::printf("per iteration: collect %.4fs  train %.4fs\n", collectT / ITERS, trainT / ITERS);
    return 0;
}
