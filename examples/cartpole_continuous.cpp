// Continuous-action CartPole (examples/CartPoleContinuous/main.cpp:23-46): the
// float Action selects the Gaussian head with a learned shared log_std.
#include <cmath>
#include <cstdio>

#include "mg/envs/cartpole_continuous.h"
#include "mg/ppo.h"

int main() {
    const uint32_t N = 4096;
    const uint32_t T = 32;

    Gym<CartPoleContinuous> gym(N);
    PPOModel<CartPoleContinuous> model(gym, 128, 4, 2, 3e-4f, T);

    for (int it = 0; it < 60; it++) {
        model.collect();
        model.train();
        if (it % 10 == 0 || it == 59) {
            uint32_t ended = 0;
            for (uint32_t t = 0; t < T; t++) {
                const uint8_t* done = model.slotDones(t);
                for (uint32_t i = 0; i < N; i++) ended += done[i];
            }
            const float meanLen = ended ? (float)(N * T) / (float)ended : (float)(N * T);
            LossStats s = model.lastStats();
            std::printf("iter %3d  steps/done %6.1f  std %.3f  entropy %.3f  kl %.4f\n", it, meanLen,
                        std::exp(model.logStdValue(0)), s.entropy, s.approxKl);
        }
    }
    return 0;
}
