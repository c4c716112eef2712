// The reference's VoxelNav training loop (examples/VoxelNav/main.cpp:30-53):
// the heightmap env with a chasm, success = an episode that ends with reward
// above 5 (it reached the goal), printed every 10 iterations.
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "mg/envs/voxelnav.h"
#include "mg/ppo.h"

int main(int argc, char** argv) {
    const uint32_t N = 4096;
    const uint32_t T = 32;
    const int iters = argc > 1 ? std::atoi(argv[1]) : 200;

    Gym<VoxelNav> gym(N);
    PPOModel<VoxelNav> model(gym, 128, 4, 2, 3e-4f, T);

    for (int it = 0; it < iters; it++) {
        model.collect();
        model.train();
        if (it % 10 == 0 || it == iters - 1) {
            uint64_t episodes = 0, successes = 0;
            for (uint32_t t = 0; t < T; t++) {
                const uint8_t* done = model.slotDones(t);
                const float* reward = model.slotRewards(t);
                for (uint32_t i = 0; i < N; i++) {
                    if (done[i]) {
                        episodes++;
                        successes += reward[i] > 5.0f;
                    }
                }
            }
            LossStats s = model.lastStats();
            std::printf("iter %3d  success %.3f  episodes %5llu  entropy %.3f\n", it,
                        episodes ? (double)successes / episodes : 0.0, (unsigned long long)episodes, s.entropy);
        }
    }
    return 0;
}
