// Host check of VoxelNav16's grid fill (include/mg/envs/voxelnav16.h): its
// reset turns each 32-bit draw into 16 cells with a multiply (bit 2 j of each
// byte of r & (r >> 1) to byte j of a word); here the grid a reset writes is
// compared with the cells read field by field from the same draws (cell
// 16 w + c occupied iff 2-bit field c of draw w is 3), for many seeds; and
// its goal-delta quotient div15(d) against the IEEE division (float)d / 15
// for every d in [-15, 15]. Prints "0 failures" on success.
#include <stdio.h>
#include <string.h>

#include "mg/envs/voxelnav16.h"

int main() {
    int fails = 0;
    uint32_t seed = 0x12345678u;
    static VoxelNav16::State s;
    for (int trial = 0; trial < 2000; ++trial) {
        const uint32_t r0 = rngNext(seed) | 1u;
        memset(&s, 0xA5, sizeof s);
        uint32_t rng = r0;
        VoxelNav16::reset(s, rng);
        // the fill's cells from the same draws, one 2-bit field at a time
        uint8_t grid[VoxelNav16::CELLS];
        uint32_t r = r0;
        for (int w = 0; w < VoxelNav16::CELLS / 16; ++w) {
            const uint32_t d = rngNext(r);
            for (int c = 0; c < 16; ++c) grid[16 * w + c] = ((d >> (2 * c)) & 3u) == 3u;
        }
        // the reset then clears at most the agent's and the goal's cells
        int diff = 0;
        for (int c = 0; c < VoxelNav16::CELLS; ++c)
            if (grid[c] != s.grid[c]) {
                const int agent = VoxelNav16::cell(s.px, s.py, s.pz), goal = VoxelNav16::cell(s.gx, s.gy, s.gz);
                if (!((c == agent || c == goal) && s.grid[c] == 0)) ++diff;
            }
        if (diff) {
            if (fails < 5) printf("fill mismatch: r0 %08x, %d cells\n", r0, diff);
            ++fails;
        }
    }
    // volatile: the reference quotient is a run-time IEEE division, not a
    // folded constant
    for (int d = -15; d <= 15; ++d) {
        volatile float x = (float)d, fifteen = 15.0f;
        const float want = x / fifteen, got = VoxelNav16::div15(d);
        if (memcmp(&want, &got, 4) != 0) {
            ++fails;
            printf("div15 mismatch: d %d, %a against %a\n", d, got, want);
        }
    }
    printf("%d failures\n", fails);
    return fails != 0;
}
