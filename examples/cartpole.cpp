// The reference's minimum training loop (examples/CartPole/main.cpp:20-36),
// unchanged apart from the includes.
#include <cstdio>

#include "mg/envs/cartpole.h"
#include "mg/ppo.h"

int main() {
    const uint32_t N = 4096;  // environments
    const uint32_t T = 32;    // steps per rollout

    Gym<CartPole> gym(N);
    PPOModel<CartPole> model(gym, 128, 4, 2, 3e-4f, T);  // embed, hidden scale, layers, lr, rollout length

    for (int it = 0; it < 40; it++) {
        model.collect();
        model.train();
        if (it % 10 == 0) {
            LossStats s = model.lastStats();
            std::printf("iter %3d  entropy %.3f  kl %.4f\n", it, s.entropy, s.approxKl);
        }
    }
    return 0;
}
