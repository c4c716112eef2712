// Training a user-defined env: Corridor's kernels come from corridor_env.hip
// (MG_DEFINE_ENV), everything else from libmetalgym_amd.
#include <cstdio>

#include "corridor.h"
#include "mg/ppo.h"

int main() {
    const uint32_t N = 1024, T = 16;
    Gym<Corridor> gym(N);
    PPOModel<Corridor> model(gym, 128, 2, 1, 1e-3f, T);
    float first = 0, last = 0;
    for (int it = 0; it < 30; it++) {
        model.collect();
        float r = 0;
        for (uint32_t t = 0; t < T; t++)
            for (uint32_t i = 0; i < N; i++) r += model.slotRewards(t)[i];
        r /= (float)(N * T);
        if (it == 0) first = r;
        last = r;
        model.train();
    }
    std::printf("corridor mean reward per step: first %.4f  last %.4f\n", first, last);
    return last > first ? 0 : 1;
}
