// TEST INFRASTRUCTURE ONLY: the CPU oracle (see oracle.h). Scalar fp32
// restatement of the reference algorithm, compiled with -ffp-contract=off and
// without fast-math. Sums run in index order; row reductions run in row order,
// so results do not depend on the thread count.
//
// Transcendentals come from include/mg/math.h, the deterministic math the
// product's env and sampler code also uses; tests pin those functions against
// libm in double precision.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../include/mg/math.h"

namespace {

template <class F>
void parallel_for(uint32_t n, int threads, F f) {
    if (threads <= 1 || n < 2) {
        f(0u, n);
        return;
    }
    uint32_t t = std::min<uint32_t>((uint32_t)threads, n);
    uint32_t chunk = (n + t - 1) / t;
    std::vector<std::thread> pool;
    for (uint32_t b = 0; b < n; b += chunk) {
        uint32_t e = std::min(n, b + chunk);
        pool.emplace_back([=]() { f(b, e); });
    }
    for (auto& th : pool) th.join();
}

// ---- rollout.h:9-29 ------------------------------------------------------
inline uint32_t xs_next(uint32_t& s) {
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}
inline float xs_unif(uint32_t& s) { return (float)(xs_next(s) >> 8) * (1.0f / 16777216.0f); }
inline float xs_unif(uint32_t& s, float lo, float hi) { return lo + (hi - lo) * xs_unif(s); }

// ---- CartPole: examples/CartPole/cartpole.metal:5-76 --------------------
struct CPState {
    float x, xDot, theta, thetaDot;
    uint32_t steps;
};
const float kGravity = 9.8f;
const float kMassPole = 0.1f;
const float kTotalMass = 1.0f + 0.1f;
const float kLength = 0.5f;
const float kPoleMassLength = 0.1f * 0.5f;
const float kForceMag = 10.0f;
const float kTau = 0.02f;
const float kThetaThreshold = 12.0f * 2.0f * 3.14159265358979323846f / 360.0f;
const float kXThreshold = 2.4f;

void cp_reset(CPState& s, uint32_t& rng) {  // cartpole.metal:37-43
    s.x = xs_unif(rng, -0.05f, 0.05f);
    s.xDot = xs_unif(rng, -0.05f, 0.05f);
    s.theta = xs_unif(rng, -0.05f, 0.05f);
    s.thetaDot = xs_unif(rng, -0.05f, 0.05f);
    s.steps = 0;
}

void cp_step(CPState& s, float force, float* obs, float& reward, uint8_t& done) {  // cartpole.metal:52-76
    float c = mg::cosf(s.theta);
    float sn = mg::sinf(s.theta);
    float temp = (force + kPoleMassLength * s.thetaDot * s.thetaDot * sn) / kTotalMass;
    float thetaAcc = (kGravity * sn - c * temp) / (kLength * (4.0f / 3.0f - kMassPole * c * c / kTotalMass));
    float xAcc = temp - kPoleMassLength * thetaAcc * c / kTotalMass;
    s.x += kTau * s.xDot;
    s.xDot += kTau * xAcc;
    s.theta += kTau * s.thetaDot;
    s.thetaDot += kTau * thetaAcc;
    s.steps += 1;
    bool terminated = std::fabs(s.x) > kXThreshold || std::fabs(s.theta) > kThetaThreshold;
    bool truncated = s.steps >= 500;
    obs[0] = s.x;
    obs[1] = s.xDot;
    obs[2] = s.theta;
    obs[3] = s.thetaDot;
    reward = 1.0f;
    done = (terminated || truncated) ? 1 : 0;
}

// ---- VoxelNav16: navigation in a 16^3 voxel grid (no reference code) -----
const int kG = 16;
const int kCells = kG * kG * kG;
struct VNState {
    int32_t px, py, pz, gx, gy, gz;
    uint32_t steps, pad;
    uint8_t grid[kCells];
};

bool vn_occ(const VNState& s, int x, int y, int z) {
    if (x < 0 || y < 0 || z < 0 || x >= kG || y >= kG || z >= kG) return true;
    return s.grid[(z * kG + y) * kG + x] != 0;
}

int vn_free_cell(VNState& s, uint32_t& rng, int avoid) {
    int c = 0;
    for (int t = 0; t < 64; ++t) {
        c = (int)(xs_next(rng) & 4095u);
        if (s.grid[c] == 0 && c != avoid) return c;
    }
    if (c == avoid) c = (c + 1) & 4095;
    s.grid[c] = 0;
    return c;
}

void vn_reset(VNState& s, uint32_t& rng) {
    for (int w = 0; w < kCells / 16; ++w) {
        uint32_t r = xs_next(rng);
        for (int j = 0; j < 16; ++j) s.grid[16 * w + j] = ((r >> (2 * j)) & 3u) == 3u ? 1 : 0;
    }
    int a = vn_free_cell(s, rng, -1);
    int g = vn_free_cell(s, rng, a);
    s.px = a % kG;
    s.py = (a / kG) % kG;
    s.pz = a / (kG * kG);
    s.gx = g % kG;
    s.gy = (g / kG) % kG;
    s.gz = g / (kG * kG);
    s.steps = 0;
}

void vn_step(VNState& s, int action, float* obs, float& reward, uint8_t& done) {
    int a = std::min(5, std::max(0, action));
    int d[3] = {0, 0, 0};
    d[a / 2] = (a % 2) ? -1 : 1;
    int nx = s.px + d[0], ny = s.py + d[1], nz = s.pz + d[2];
    bool blocked = vn_occ(s, nx, ny, nz);
    if (!blocked) {
        s.px = nx;
        s.py = ny;
        s.pz = nz;
    }
    s.steps += 1;
    bool goal = s.px == s.gx && s.py == s.gy && s.pz == s.gz;
    reward = goal ? 1.0f : (blocked ? -0.1f : -0.01f);
    done = (goal || s.steps >= 256) ? 1 : 0;
    int k = 0;
    for (int dz = -1; dz <= 1; ++dz)
        for (int dy = -1; dy <= 1; ++dy)
            for (int dx = -1; dx <= 1; ++dx) obs[k++] = vn_occ(s, s.px + dx, s.py + dy, s.pz + dz) ? 1.0f : 0.0f;
    obs[27] = (float)(s.gx - s.px) / 15.0f;
    obs[28] = (float)(s.gy - s.py) / 15.0f;
    obs[29] = (float)(s.gz - s.pz) / 15.0f;
}

// ---- VoxelNav: examples/VoxelNav/voxelnav.metal:9-174 ----------------------
// Heightmap 32 x 32 (index cx * 32 + cz), 8 x 4 depth rays, 6 actions. The
// reference's Metal cos / sin are replaced by mg::cosf / mg::sinf (the
// product's deterministic functions).
const int kVW = 32;
const float kVPi = 3.14159265358979323846f;
const float kVFov = 90.0f * kVPi / 180.0f;
const float kVMaxDepth = 24.0f;
struct VRState {
    float x, z, yaw, gx, gz, prevDist;
    uint32_t steps, cobble;
    uint8_t height[kVW * kVW];
};

bool vr_inside(int cx, int cz) { return cx >= 0 && cz >= 0 && cx < kVW && cz < kVW; }

float vr_height(const VRState& s, float x, float z) {  // voxelnav.metal:40-43
    int cx = (int)std::floor(x), cz = (int)std::floor(z);
    return vr_inside(cx, cz) ? (float)s.height[cx * kVW + cz] : 0.0f;
}

float vr_dist(const VRState& s) {  // voxelnav.metal:44-47
    float dx = s.gx - s.x, dz = s.gz - s.z;
    return std::sqrt(dx * dx + dz * dz);
}

float vr_lerp(float a, float b, float t) { return a + (b - a) * t; }  // Metal mix()

void vr_reset(VRState& s, uint32_t& rng) {  // voxelnav.metal:49-83
    float knot[25];
    for (int i = 0; i < 25; ++i) knot[i] = xs_unif(rng, 3.0f, 9.0f);
    for (int cx = 0; cx < kVW; ++cx) {
        float fx = (float)cx / (float)(kVW - 1) * 4.0f;
        int ix = std::min((int)fx, 3);
        float tx = fx - (float)ix;
        for (int cz = 0; cz < kVW; ++cz) {
            float fz = (float)cz / (float)(kVW - 1) * 4.0f;
            int iz = std::min((int)fz, 3);
            float tz = fz - (float)iz;
            float lo = vr_lerp(knot[ix * 5 + iz], knot[(ix + 1) * 5 + iz], tx);
            float hi = vr_lerp(knot[ix * 5 + iz + 1], knot[(ix + 1) * 5 + iz + 1], tx);
            s.height[cx * kVW + cz] = (uint8_t)std::round(vr_lerp(lo, hi, tz));
        }
    }
    uint32_t width = 2 + xs_next(rng) % 4u;
    uint32_t left = 12 + xs_next(rng) % 6u;
    uint32_t lift = xs_next(rng) % 3u;
    for (uint32_t cx = 0; cx < (uint32_t)kVW; ++cx)
        for (int cz = 0; cz < kVW; ++cz) {
            uint8_t& h = s.height[cx * kVW + cz];
            if (cx >= left && cx < left + width)
                h = 0;
            else if (cx >= left + width)
                h = (uint8_t)std::min<uint32_t>(h + lift, 15u);
        }
    s.x = 2.5f + xs_unif(rng) * (float)(left - 4);
    s.z = 2.5f + xs_unif(rng) * (float)(kVW - 5);
    s.gx = (float)(left + width) + 2.5f + xs_unif(rng) * (float)(kVW - 5 - (int)(left + width));
    s.gz = 2.5f + xs_unif(rng) * (float)(kVW - 5);
    s.yaw = xs_unif(rng, -kVPi, kVPi);
    s.prevDist = vr_dist(s);
    s.steps = 0;
    s.cobble = 16;
}

void vr_observe(const VRState& s, float* obs) {  // voxelnav.metal:85-115
    static const float pitchDeg[4] = {-45.0f, -20.0f, 0.0f, 15.0f};
    float h = vr_height(s, s.x, s.z);
    float eye = h + 1.6f;
    for (int c = 0; c < 8; ++c) {
        float a = s.yaw + ((float)c / 7.0f - 0.5f) * kVFov;
        float cosA = mg::cosf(a), sinA = mg::sinf(a);
        for (int r = 0; r < 4; ++r) {
            float p = pitchDeg[r] * kVPi / 180.0f;
            float cosP = mg::cosf(p);
            float dx = cosP * cosA, dy = mg::sinf(p), dz = cosP * sinA;
            float depth = kVMaxDepth;
            for (float t = 0.5f; t < kVMaxDepth; t += 0.5f) {
                float px = s.x + t * dx, py = eye + t * dy, pz = s.z + t * dz;
                int cx = (int)std::floor(px), cz = (int)std::floor(pz);
                if (!vr_inside(cx, cz) || py <= (float)s.height[cx * kVW + cz]) {
                    depth = t;
                    break;
                }
            }
            obs[c * 4 + r] = depth / kVMaxDepth;
        }
    }
    float gx = s.gx - s.x, gz = s.gz - s.z;
    float cy = mg::cosf(s.yaw), sy = mg::sinf(s.yaw);
    obs[32] = (gx * cy + gz * sy) / (float)kVW;
    obs[33] = (-gx * sy + gz * cy) / (float)kVW;
    obs[34] = (vr_height(s, s.gx, s.gz) - h) / 8.0f;
    obs[35] = std::sqrt(gx * gx + gz * gz) / (float)kVW;
    obs[36] = sy;
    obs[37] = cy;
    obs[38] = (float)s.cobble / 16.0f;
    obs[39] = h / 16.0f;
}

// voxelnav.metal:119-129; true when the move ends in the void
bool vr_move(VRState& s, float nx, float nz) {
    int cx = (int)std::floor(nx), cz = (int)std::floor(nz);
    if (!vr_inside(cx, cz)) return false;
    float here = vr_height(s, s.x, s.z);
    float there = (float)s.height[cx * kVW + cz];
    if (there != 0.0f && there > here + 1.0f) return false;
    s.x = nx;
    s.z = nz;
    return there == 0.0f;
}

void vr_step(VRState& s, int action, float* obs, float& reward, uint8_t& done) {  // voxelnav.metal:131-162
    float cy = mg::cosf(s.yaw), sy = mg::sinf(s.yaw);
    bool fell = false;
    if (action == 0) {
        fell = vr_move(s, s.x + cy, s.z + sy);
    } else if (action == 1) {
        fell = vr_move(s, s.x - cy, s.z - sy);
    } else if (action == 2) {
        s.yaw -= kVPi / 6.0f;
    } else if (action == 3) {
        s.yaw += kVPi / 6.0f;
    } else if (action == 4) {
        fell = vr_move(s, s.x + 2.0f * cy, s.z + 2.0f * sy);
    } else if (action == 5) {
        int cx = (int)std::floor(s.x + cy), cz = (int)std::floor(s.z + sy);
        if (s.cobble > 0 && vr_inside(cx, cz)) {
            uint8_t& t = s.height[cx * kVW + cz];
            uint32_t here = (uint32_t)vr_height(s, s.x, s.z);
            if (t == 0) {
                t = (uint8_t)here;
                s.cobble -= 1;
            } else if ((uint32_t)t <= here) {
                t = (uint8_t)(t + 1);
                s.cobble -= 1;
            }
        }
    }
    if (s.yaw > kVPi) s.yaw -= 2.0f * kVPi;
    if (s.yaw < -kVPi) s.yaw += 2.0f * kVPi;
    s.steps += 1;
    float d = vr_dist(s);
    float progress = std::min(1.5f, std::max(-1.5f, s.prevDist - d));
    reward = -0.05f + 0.2f * progress;
    s.prevDist = d;
    bool success = d < 1.5f;
    if (success) reward += 10.0f;
    if (fell) reward -= 5.0f;
    done = (success || fell || s.steps >= 250) ? 1 : 0;
    vr_observe(s, obs);
}

// ---- env dispatch -----------------------------------------------------------
orc_env_info env_info(int env) {
    switch (env) {
        case ORC_CARTPOLE: return {sizeof(CPState), 4, 4, 2, 0};
        case ORC_CARTPOLE_CONT:
        case ORC_CARTPOLE_CONT_CLAMP: return {sizeof(CPState), 4, 4, 1, 1};
        case ORC_VOXELNAV16: return {sizeof(VNState), 4, 30, 6, 0};
        case ORC_VOXELNAV: return {sizeof(VRState), 4, 40, 6, 0};
        default: return {0, 0, 0, 0, 0};
    }
}

void env_reset(int env, void* state, uint32_t& rng) {
    if (env == ORC_VOXELNAV16)
        vn_reset(*static_cast<VNState*>(state), rng);
    else if (env == ORC_VOXELNAV)
        vr_reset(*static_cast<VRState*>(state), rng);
    else
        cp_reset(*static_cast<CPState*>(state), rng);
}

void env_step(int env, void* state, const void* action, float* obs, float& reward, uint8_t& done) {
    switch (env) {
        case ORC_CARTPOLE: {
            int a;
            std::memcpy(&a, action, 4);
            cp_step(*static_cast<CPState*>(state), a == 1 ? kForceMag : -kForceMag, obs, reward, done);
            break;
        }
        case ORC_CARTPOLE_CONT: {  // force = 10 tanh(a)
            float a;
            std::memcpy(&a, action, 4);
            cp_step(*static_cast<CPState*>(state), kForceMag * mg::tanhf(a), obs, reward, done);
            break;
        }
        case ORC_CARTPOLE_CONT_CLAMP: {  // cartpole_continuous.metal:57
            float a;
            std::memcpy(&a, action, 4);
            float c = a < -1.0f ? -1.0f : (a > 1.0f ? 1.0f : a);
            cp_step(*static_cast<CPState*>(state), c * kForceMag, obs, reward, done);
            break;
        }
        case ORC_VOXELNAV16: {
            int a;
            std::memcpy(&a, action, 4);
            vn_step(*static_cast<VNState*>(state), a, obs, reward, done);
            break;
        }
        case ORC_VOXELNAV: {
            int a;
            std::memcpy(&a, action, 4);
            vr_step(*static_cast<VRState*>(state), a, obs, reward, done);
            break;
        }
    }
}

// A random action drawn from the env's stream (this build's random policy):
// rngInt(rng, ACT_DIM) for a discrete action, uniform [-1, 1) per dimension
// for a float action.
void random_action(int env, uint32_t& rng, void* out) {
    orc_env_info info = env_info(env);
    if (info.continuous) {
        float* f = static_cast<float*>(out);
        for (uint32_t k = 0; k < info.act_dim; ++k) f[k] = xs_unif(rng, -1.0f, 1.0f);
    } else {
        int a = (int)(xs_next(rng) % info.act_dim);
        std::memcpy(out, &a, 4);
    }
}

// ---- parameters ----------------------------------------------------------
uint32_t pad128(uint32_t x) { return (x + 127u) / 128u * 128u; }

orc_layout make_layout(const orc_dims& d) {
    orc_layout L;
    std::memset(&L, 0, sizeof(L));
    const uint32_t E = d.embed, H = d.hidden, O = d.obs_dim, A = d.act_dim;
    uint32_t off = 0;
    L.head_dim = A + 1;
    L.off_in_w = off, off += pad128(O * E);
    L.off_in_b = off, off += pad128(E);
    for (uint32_t n = 0; n <= d.layers; ++n) {
        L.off_ln_gamma[n] = off, off += pad128(E);
        L.off_ln_beta[n] = off, off += pad128(E);
    }
    if (d.continuous) L.off_log_std = off, off += pad128(A);
    L.float_group = off;
    for (uint32_t n = 0; n < d.layers; ++n) {
        L.off_up[n] = off, off += pad128(E * H);
        L.off_down[n] = off, off += pad128(H * E);
    }
    L.off_head = off, off += pad128(E * L.head_dim);
    L.count = off;
    return L;
}

uint64_t splitmix(uint64_t& s) {  // SplitMix64 (Steele, Lea & Flood 2014)
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
const uint64_t kInitStream = 0x4D47494E49540000ull;     // "MGINIT"
const uint64_t kShuffleStream = 0x4D47534855460000ull;  // "MGSHUF"

float uniform_pm(uint64_t& s, float bound) {
    float u = (float)(splitmix(s) >> 40) * (1.0f / 16777216.0f);
    return bound * (2.0f * u - 1.0f);
}

// ---- forward: model/ppo.h:575-626 and the kernels it encodes -------------
struct Net {
    orc_dims d;
    orc_layout L;
    const float* P;
    uint32_t E, H, O, A, HD, NL;
    explicit Net(const orc_dims& dims, const float* params) : d(dims), L(make_layout(dims)), P(params) {
        E = d.embed, H = d.hidden, O = d.obs_dim, A = d.act_dim, HD = A + 1, NL = d.layers;
    }
};

// model/layernorm.metal:10-71 (two-pass mean and population variance)
void ln_forward(const float* h, const float* gamma, const float* beta, uint32_t E, float* xn, float* x, float* stdev) {
    float sum = 0.0f;
    for (uint32_t c = 0; c < E; ++c) sum += h[c];
    float mean = sum / (float)E;
    float var = 0.0f;
    for (uint32_t c = 0; c < E; ++c) {
        float dlt = h[c] - mean;
        var += dlt * dlt;
    }
    var /= (float)E;
    float sd = std::sqrt(var + 1e-5f);
    float rstd = 1.0f / sd;
    *stdev = sd;
    for (uint32_t c = 0; c < E; ++c) {
        float v = (h[c] - mean) * rstd;
        xn[c] = v;
        x[c] = gamma[c] * v + beta[c];
    }
}

// bfloat16 rounding of an fp32 value (round to nearest, ties to even), kept as
// the float it represents: the matrix operands of the reference's matmuls
// (model/mlp.metal:43-48, 80-85 multiply bfloat16 tiles).
float round_bf16(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

// Per-row activation record for the backward pass.
struct Acts {
    std::vector<float> xn, x, sd, v;  // xn/x: [(L+1)][E], sd: [L+1], v: [L][H]
    void init(const Net& n) {
        xn.assign((n.NL + 1) * n.E, 0.0f);
        x.assign((n.NL + 1) * n.E, 0.0f);
        sd.assign(n.NL + 1, 0.0f);
        v.assign(n.NL * n.H, 0.0f);
    }
};

// relu_mask ([L][H], nullable) replaces the ReLU's decision v > 0 for this
// row: a unit passes (v = z) where the mask is 1 and is 0 where it is 0.
// z_out ([L][H], nullable) receives the pre-activations z.
void forward_row(const Net& n, const float* obs, float* head, float* xn_out, float* x_out, float* sd_out,
                 float* v_out, const uint8_t* relu_mask = nullptr, float* z_out = nullptr) {
    const uint32_t E = n.E, H = n.H;
    std::vector<float> h(E), xn(E), x(E), v(H), out(E);
    // model/input.metal:11-27: acc = bias, then obs . W in k order
    const float* W = n.P + n.L.off_in_w;
    const float* b = n.P + n.L.off_in_b;
    for (uint32_t c = 0; c < E; ++c) h[c] = b[c];
    for (uint32_t k = 0; k < n.O; ++k)
        for (uint32_t c = 0; c < E; ++c) h[c] += obs[k] * W[k * E + c];
    for (uint32_t l = 0; l < n.NL; ++l) {
        float sd;
        ln_forward(h.data(), n.P + n.L.off_ln_gamma[l], n.P + n.L.off_ln_beta[l], E, xn.data(), x.data(), &sd);
        const bool bf = n.d.bf16 != 0;
        if (xn_out) std::memcpy(xn_out + l * E, xn.data(), E * 4);
        if (x_out)  // the up GEMM's operand (rounded in bf16 mode), for dUp
            for (uint32_t k = 0; k < E; ++k) x_out[l * E + k] = bf ? round_bf16(x[k]) : x[k];
        if (sd_out) sd_out[l] = sd;
        // model/mlp.metal:18-58: V = X Up, relu (bf16 operands: X and Up rounded)
        const float* Up = n.P + n.L.off_up[l];
        std::fill(v.begin(), v.end(), 0.0f);
        for (uint32_t k = 0; k < E; ++k) {
            float xk = bf ? round_bf16(x[k]) : x[k];
            const float* row = Up + (size_t)k * H;
            if (bf)
                for (uint32_t j = 0; j < H; ++j) v[j] += xk * round_bf16(row[j]);
            else
                for (uint32_t j = 0; j < H; ++j) v[j] += xk * row[j];
        }
        if (z_out) std::memcpy(z_out + (size_t)l * H, v.data(), H * 4);
        if (relu_mask)
            for (uint32_t j = 0; j < H; ++j) v[j] = relu_mask[(size_t)l * H + j] ? v[j] : 0.0f;
        else
            for (uint32_t j = 0; j < H; ++j) v[j] = v[j] > 0.0f ? v[j] : 0.0f;
        if (v_out)  // the down GEMM's operand (rounded in bf16 mode), for dDown and the relu mask
            for (uint32_t j = 0; j < H; ++j) v_out[(size_t)l * H + j] = bf ? round_bf16(v[j]) : v[j];
        // model/mlp.metal:60-86: Out = V Down (bf16 operands: V and Down rounded);
        // model/elementwise.metal:4-13 residual add
        const float* Dn = n.P + n.L.off_down[l];
        std::fill(out.begin(), out.end(), 0.0f);
        for (uint32_t j = 0; j < H; ++j) {
            float vj = bf ? round_bf16(v[j]) : v[j];
            const float* row = Dn + (size_t)j * E;
            if (bf)
                for (uint32_t c = 0; c < E; ++c) out[c] += vj * round_bf16(row[c]);
            else
                for (uint32_t c = 0; c < E; ++c) out[c] += vj * row[c];
        }
        for (uint32_t c = 0; c < E; ++c) h[c] = h[c] + out[c];
    }
    float sd;
    ln_forward(h.data(), n.P + n.L.off_ln_gamma[n.NL], n.P + n.L.off_ln_beta[n.NL], E, xn.data(), x.data(), &sd);
    if (xn_out) std::memcpy(xn_out + n.NL * E, xn.data(), E * 4);
    if (x_out) std::memcpy(x_out + n.NL * E, x.data(), E * 4);
    if (sd_out) sd_out[n.NL] = sd;
    // model/linear.metal:17-37: head = X W (no bias)
    const float* Wh = n.P + n.L.off_head;
    for (uint32_t j = 0; j < n.HD; ++j) head[j] = 0.0f;
    for (uint32_t k = 0; k < E; ++k)
        for (uint32_t j = 0; j < n.HD; ++j) head[j] += x[k] * Wh[k * n.HD + j];
}

const float kLogSqrt2Pi = 0.9189385332046727f;
const float kPiF = 3.14159265358979323846f;

// model/sample.metal:18-47. Returns the chosen action.
int sample_categorical(const float* h, uint32_t A, uint32_t& rng, float* logp) {
    float rowMax = -INFINITY;
    for (uint32_t a = 0; a < A; ++a) rowMax = std::max(rowMax, h[a]);
    float sum = 0.0f;
    for (uint32_t a = 0; a < A; ++a) sum += mg::expf(h[a] - rowMax);
    float lse = rowMax + mg::logf(sum);
    float u = (float)(xs_next(rng) >> 8) * (1.0f / 16777216.0f) * sum;
    uint32_t chosen = A - 1;
    float acc = 0.0f;
    for (uint32_t a = 0; a < A; ++a) {
        acc += mg::expf(h[a] - rowMax);
        if (u < acc) {
            chosen = a;
            break;
        }
    }
    *logp = h[chosen] - lse;
    return (int)chosen;
}

float categorical_logp(const float* h, uint32_t A, int a) {
    float rowMax = -INFINITY;
    for (uint32_t j = 0; j < A; ++j) rowMax = std::max(rowMax, h[j]);
    float sum = 0.0f;
    for (uint32_t j = 0; j < A; ++j) sum += mg::expf(h[j] - rowMax);
    return h[a] - (rowMax + mg::logf(sum));
}

// model/gaussian.metal:22-71 (Box-Muller pairs)
void sample_gaussian(const float* h, const float* logStd, uint32_t A, uint32_t& rng, float* act, float* logp) {
    float lp = 0.0f, z0 = 0.0f, z1 = 0.0f;
    for (uint32_t k = 0; k < A; ++k) {
        if ((k & 1u) == 0u) {
            float u1 = 1.0f - (float)(xs_next(rng) >> 8) * (1.0f / 16777216.0f);
            float u2 = (float)(xs_next(rng) >> 8) * (1.0f / 16777216.0f);
            float r = std::sqrt(-2.0f * mg::logf(u1));
            float th = 2.0f * kPiF * u2;
            z0 = r * mg::cosf(th);
            z1 = r * mg::sinf(th);
        }
        float zk = (k & 1u) ? z1 : z0;
        float ls = logStd[k];
        float mu = h[k];
        float a = mu + mg::expf(ls) * zk;
        float dd = (a - mu) * mg::expf(-ls);
        act[k] = a;
        lp += -0.5f * dd * dd - ls - kLogSqrt2Pi;
    }
    *logp = lp;
}

float gaussian_logp(const float* h, const float* logStd, uint32_t A, const float* act) {
    float lp = 0.0f;
    for (uint32_t k = 0; k < A; ++k) {
        float ls = logStd[k];
        float dd = (act[k] - h[k]) * mg::expf(-ls);
        lp += -0.5f * dd * dd - ls - kLogSqrt2Pi;
    }
    return lp;
}

// model/layernorm.metal:74-127 for one row: dZ is the gradient at the LN
// output; returns dX in dx (the reference writes it in place).
void ln_backward(const float* dZ, const float* xn, const float* gamma, float sd, uint32_t E, float* dx) {
    std::vector<float> dxn(E);
    for (uint32_t i = 0; i < E; ++i) dxn[i] = dZ[i] * gamma[i];
    float s1 = 0.0f, s2 = 0.0f;
    for (uint32_t i = 0; i < E; ++i) {
        s1 += dxn[i];
        s2 += dxn[i] * xn[i];
    }
    float r1 = s1 / (float)E, r2 = s2 / (float)E, rd = 1.0f / sd;
    for (uint32_t i = 0; i < E; ++i) dx[i] = rd * (dxn[i] - r1 - xn[i] * r2);
}

}  // namespace

// ============================================================================
extern "C" {

uint32_t orc_rng_next(uint32_t* s) { return xs_next(*s); }
float orc_rng_uniform(uint32_t* s) { return xs_unif(*s); }
float orc_rng_uniform_range(uint32_t* s, float lo, float hi) { return xs_unif(*s, lo, hi); }
uint32_t orc_rng_int(uint32_t* s, uint32_t n) { return xs_next(*s) % n; }

float orc_round_bf16(float x) { return round_bf16(x); }
float orc_expf(float x) { return mg::expf(x); }
float orc_logf(float x) { return mg::logf(x); }
float orc_sinf(float x) { return mg::sinf(x); }
float orc_cosf(float x) { return mg::cosf(x); }
float orc_tanhf(float x) { return mg::tanhf(x); }

int orc_env_info_get(int env, orc_env_info* out) {
    *out = env_info(env);
    return out->state_bytes ? 0 : -1;
}

void orc_env_reset(int env, void* state, uint32_t* rng) { env_reset(env, state, *rng); }

void orc_env_step(int env, void* state, const void* action, float* obs, float* reward, uint8_t* done) {
    env_step(env, state, action, obs, *reward, *done);
}

// gym.h:54-61: done = 1, actions = 0, rng = seed hash (seed 0 = reference)
void orc_gym_init(int env, uint32_t n, uint32_t seed, void* state, uint32_t* rng, uint8_t* done, void* actions) {
    orc_env_info info = env_info(env);
    std::memset(state, 0, (size_t)n * info.state_bytes);
    std::memset(done, 1, n);
    std::memset(actions, 0, (size_t)n * info.action_bytes);
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t s = (i * 2654435761u + 1u) ^ (seed * 0x9E3779B9u);
        rng[i] = s ? s : 0x6D2B79F5u;
    }
}

// rollout.h:31-54, `steps` times per env
void orc_rollout(int env, uint32_t n, uint32_t steps, int random, void* state, uint32_t* rng, uint8_t* done,
                 const void* actions_in, void* actions_out, float* obs_out, float* reward_out, uint8_t* done_out,
                 int threads) {
    orc_env_info info = env_info(env);
    parallel_for(n, threads, [&](uint32_t b, uint32_t e) {
        std::vector<float> obs(info.obs_dim);
        uint8_t act[64];
        for (uint32_t i = b; i < e; ++i) {
            char* s = static_cast<char*>(state) + (size_t)i * info.state_bytes;
            for (uint32_t t = 0; t < steps; ++t) {
                size_t k = (size_t)t * n + i;
                if (random) {
                    random_action(env, rng[i], act);
                    if (actions_out) std::memcpy(static_cast<char*>(actions_out) + k * info.action_bytes, act,
                                                 info.action_bytes);
                } else {
                    std::memcpy(act, static_cast<const char*>(actions_in) + k * info.action_bytes, info.action_bytes);
                }
                if (done[i]) env_reset(env, s, rng[i]);
                float r = 0.0f;
                std::fill(obs.begin(), obs.end(), 0.0f);
                env_step(env, s, act, obs.data(), r, done[i]);
                if (obs_out) std::memcpy(obs_out + k * info.obs_dim, obs.data(), info.obs_dim * 4);
                if (reward_out) reward_out[k] = r;
                if (done_out) done_out[k] = done[i];
            }
        }
    });
}

int orc_layout_get(const orc_dims* d, orc_layout* out) {
    *out = make_layout(*d);
    return 0;
}

uint64_t orc_splitmix_next(uint64_t* state) { return splitmix(*state); }

// model/ppo.h:375-410, drawn from SplitMix64 instead of the reference's
// generator: uniform init with the reference's per-layer std
// (bound = sqrt(3) std), drawn in the reference's parameter order.
void orc_init_params(const orc_dims* dp, uint32_t seed, float* P) {
    const orc_dims& d = *dp;
    orc_layout L = make_layout(d);
    std::memset(P, 0, (size_t)L.count * 4);
    uint64_t s = kInitStream ^ (uint64_t)seed;
    const uint32_t E = d.embed, H = d.hidden, O = d.obs_dim, A = d.act_dim, HD = A + 1;
    float bIn = std::sqrt(3.0f / (float)O);
    for (uint32_t i = 0; i < O * E; ++i) P[L.off_in_w + i] = uniform_pm(s, bIn);
    for (uint32_t l = 0; l < d.layers; ++l) {
        for (uint32_t c = 0; c < E; ++c) P[L.off_ln_gamma[l] + c] = 1.0f;
        float bUp = std::sqrt(6.0f / (float)E);
        for (uint32_t i = 0; i < E * H; ++i) P[L.off_up[l] + i] = uniform_pm(s, bUp);
        float bDn = std::sqrt(3.0f / (float)H) / std::sqrt((float)d.layers);
        for (uint32_t i = 0; i < H * E; ++i) P[L.off_down[l] + i] = uniform_pm(s, bDn);
    }
    for (uint32_t c = 0; c < E; ++c) P[L.off_ln_gamma[d.layers] + c] = 1.0f;
    float bPol = 0.01f * std::sqrt(3.0f), bVal = std::sqrt(3.0f / (float)E);
    for (uint32_t k = 0; k < E; ++k)
        for (uint32_t j = 0; j < HD; ++j) P[L.off_head + k * HD + j] = uniform_pm(s, j < A ? bPol : bVal);
    // log_std starts at 0 (model/ppo.h:115, 408-410): already zero
}

void orc_forward(const orc_dims* d, const float* params, const float* obs, uint32_t rows, float* head, int threads) {
    Net net(*d, params);
    parallel_for(rows, threads, [&](uint32_t b, uint32_t e) {
        for (uint32_t r = b; r < e; ++r)
            forward_row(net, obs + (size_t)r * net.O, head + (size_t)r * net.HD, nullptr, nullptr, nullptr, nullptr);
    });
}

void orc_sample(const orc_dims* d, const float* params, const float* head, uint32_t rows, uint32_t* rng,
                void* actions, float* logp, float* value) {
    Net net(*d, params);
    for (uint32_t r = 0; r < rows; ++r) {
        const float* h = head + (size_t)r * net.HD;
        if (d->continuous) {
            sample_gaussian(h, params + net.L.off_log_std, net.A, rng[r], static_cast<float*>(actions) + r * net.A,
                            &logp[r]);
        } else {
            static_cast<int*>(actions)[r] = sample_categorical(h, net.A, rng[r], &logp[r]);
        }
        value[r] = h[net.A];
    }
}

void orc_gae(const float* reward, const uint8_t* done, const float* value, const float* head, uint32_t head_dim,
             uint32_t act_dim, uint32_t n, uint32_t horizon, float gamma, float lambda, float* adv, float* ret) {
    for (uint32_t i = 0; i < n; ++i) {  // model/gae.metal:14-36
        float lastAdv = 0.0f;
        float nextValue = head[(size_t)i * head_dim + act_dim];
        for (int t = (int)horizon - 1; t >= 0; --t) {
            size_t k = (size_t)t * n + i;
            float nonTerminal = done[k] ? 0.0f : 1.0f;
            float delta = reward[k] + gamma * nextValue * nonTerminal - value[k];
            lastAdv = delta + gamma * lambda * nonTerminal * lastAdv;
            adv[k] = lastAdv;
            ret[k] = lastAdv + value[k];
            nextValue = value[k];
        }
    }
}

void orc_collect(int env, const orc_dims* d, const float* params, uint32_t n, uint32_t horizon, int first,
                 float gamma, float lambda, void* state, uint32_t* rng, uint8_t* done, float* obs_slots,
                 void* action_slots, float* logp_slots, float* value_slots, float* reward_slots,
                 uint8_t* done_slots, float* adv_slots, float* ret_slots, float* head_out,
                 const void* teacher_actions, void* sampled_actions, int threads) {
    Net net(*d, params);
    orc_env_info info = env_info(env);
    const uint32_t O = net.O, A = net.A, HD = net.HD;
    const size_t ab = info.action_bytes;
    const float* logStd = d->continuous ? params + net.L.off_log_std : nullptr;
    parallel_for(n, threads, [&](uint32_t b, uint32_t e) {
        std::vector<float> head(HD), obs(O);
        uint8_t act[64], own[64];
        for (uint32_t i = b; i < e; ++i) {
            char* s = static_cast<char*>(state) + (size_t)i * info.state_bytes;
            if (first) {  // model/ppo.h:720-722: one step with the zeroed action slot 0
                std::memset(act, 0, sizeof(act));
                if (done[i]) env_reset(env, s, rng[i]);
                float r = 0.0f;
                std::fill(obs.begin(), obs.end(), 0.0f);
                env_step(env, s, act, obs.data(), r, done[i]);
                std::memcpy(obs_slots + (size_t)i * O, obs.data(), O * 4);
                reward_slots[i] = r;
            } else {  // model/ppo.h:724
                std::memcpy(obs_slots + (size_t)i * O, obs_slots + ((size_t)horizon * n + i) * O, O * 4);
            }
            for (uint32_t t = 0; t < horizon; ++t) {  // model/ppo.h:727-733
                size_t k = (size_t)t * n + i;
                forward_row(net, obs_slots + k * O, head.data(), nullptr, nullptr, nullptr, nullptr);
                float lp;
                if (d->continuous) {
                    sample_gaussian(head.data(), logStd, A, rng[i], reinterpret_cast<float*>(own), &lp);
                } else {
                    int a = sample_categorical(head.data(), A, rng[i], &lp);
                    std::memcpy(own, &a, 4);
                }
                if (sampled_actions) std::memcpy(static_cast<char*>(sampled_actions) + k * ab, own, ab);
                if (teacher_actions) {
                    std::memcpy(act, static_cast<const char*>(teacher_actions) + k * ab, ab);
                    if (d->continuous)
                        lp = gaussian_logp(head.data(), logStd, A, reinterpret_cast<const float*>(act));
                    else {
                        int a;
                        std::memcpy(&a, act, 4);
                        lp = categorical_logp(head.data(), A, a);
                    }
                } else {
                    std::memcpy(act, own, ab);
                }
                std::memcpy(static_cast<char*>(action_slots) + k * ab, act, ab);
                logp_slots[k] = lp;
                value_slots[k] = head[A];
                if (done[i]) env_reset(env, s, rng[i]);
                float r = 0.0f;
                std::fill(obs.begin(), obs.end(), 0.0f);
                env_step(env, s, act, obs.data(), r, done[i]);
                std::memcpy(obs_slots + ((size_t)(t + 1) * n + i) * O, obs.data(), O * 4);
                reward_slots[k] = r;
                done_slots[k] = done[i];
            }
            // model/ppo.h:735: bootstrap forward on obs[T]
            forward_row(net, obs_slots + ((size_t)horizon * n + i) * O, head_out + (size_t)i * HD, nullptr, nullptr,
                        nullptr, nullptr);
        }
    });
    orc_gae(reward_slots, done_slots, value_slots, head_out, HD, A, n, horizon, gamma, lambda, adv_slots, ret_slots);
}

void orc_train_minibatch(const orc_dims* dp, const orc_hparams* hp, float* P, float* M, float* V, uint32_t step,
                         uint32_t B, const float* obs, const void* actions, const float* adv, const float* ret,
                         const float* old_logp, float* grad_out, orc_stats* stats, float* head_out, int threads) {
    orc_train_minibatch_masked(dp, hp, P, M, V, step, B, obs, actions, adv, ret, old_logp, grad_out, stats, head_out,
                               nullptr, nullptr, threads);
}

void orc_train_minibatch_masked(const orc_dims* dp, const orc_hparams* hp, float* P, float* M, float* V,
                                uint32_t step, uint32_t B, const float* obs, const void* actions, const float* adv,
                                const float* ret, const float* old_logp, float* grad_out, orc_stats* stats,
                                float* head_out, const uint8_t* relu_mask, float* preact_out, int threads) {
    const orc_dims& d = *dp;
    Net net(d, P);
    const orc_layout& L = net.L;
    const uint32_t E = net.E, H = net.H, O = net.O, A = net.A, HD = net.HD, NL = net.NL;
    const size_t actW = (size_t)(NL + 1) * E;

    // forward with activation capture (model/ppo.h:909)
    std::vector<float> head((size_t)B * HD), xn((size_t)B * actW), x((size_t)B * actW), sd((size_t)B * (NL + 1)),
        vv((size_t)B * NL * H);
    parallel_for(B, threads, [&](uint32_t b, uint32_t e) {
        for (uint32_t r = b; r < e; ++r)
            forward_row(net, obs + (size_t)r * O, &head[(size_t)r * HD], &xn[r * actW], &x[r * actW],
                        &sd[(size_t)r * (NL + 1)], &vv[(size_t)r * NL * H],
                        relu_mask ? relu_mask + (size_t)r * NL * H : nullptr,
                        preact_out ? preact_out + (size_t)r * NL * H : nullptr);
    });
    // the backward's relu derivative: the forward's decision (the mask, if given)
    auto passes = [&](uint32_t r, uint32_t l, uint32_t j) {
        const size_t k = ((size_t)r * NL + l) * H + j;
        return relu_mask ? relu_mask[k] != 0 : vv[k] > 0.0f;
    };
    if (head_out) std::memcpy(head_out, head.data(), head.size() * 4);

    // model/gae.metal:42-77 over the minibatch rows
    float sum = 0.0f;
    for (uint32_t r = 0; r < B; ++r) sum += adv[r];
    float mean = sum / (float)B;
    float var = 0.0f;
    for (uint32_t r = 0; r < B; ++r) {
        float dl = adv[r] - mean;
        var += dl * dl;
    }
    var = var / (float)B;
    float inv = 1.0f / (std::sqrt(var) + 1e-8f);

    // loss + head gradient per row
    const float scale = 1.0f / (float)B;
    std::vector<float> dhead((size_t)B * HD, 0.0f), rowStats((size_t)B * 5), dls((size_t)B * (A ? A : 1), 0.0f);
    const float* logStd = d.continuous ? P + L.off_log_std : nullptr;
    for (uint32_t r = 0; r < B; ++r) {
        const float* h = &head[(size_t)r * HD];
        float* dz = &dhead[(size_t)r * HD];
        float a_n = (adv[r] - mean) * inv;
        float entropy = 0.0f, logpA, ratio, policyLoss, gLogp;
        if (!d.continuous) {  // model/policy.metal:14-69
            float rowMax = -INFINITY;
            for (uint32_t j = 0; j < A; ++j) rowMax = std::max(rowMax, h[j]);
            float s = 0.0f;
            for (uint32_t j = 0; j < A; ++j) s += mg::expf(h[j] - rowMax);
            float lse = rowMax + mg::logf(s);
            for (uint32_t j = 0; j < A; ++j) {
                float lp = h[j] - lse;
                entropy -= mg::expf(lp) * lp;
            }
            int a = static_cast<const int*>(actions)[r];
            logpA = h[a] - lse;
            ratio = mg::expf(logpA - old_logp[r]);
            float surr1 = ratio * a_n;
            float cr = std::min(std::max(ratio, 1.0f - hp->clip), 1.0f + hp->clip);
            float surr2 = cr * a_n;
            policyLoss = -std::min(surr1, surr2);
            gLogp = (surr1 <= surr2) ? -a_n * ratio : 0.0f;
            for (uint32_t j = 0; j < A; ++j) {
                float lp = h[j] - lse;
                float prob = mg::expf(lp);
                float g = gLogp * (((int)j == a ? 1.0f : 0.0f) - prob) + hp->entropy_coef * prob * (lp + entropy);
                dz[j] = g * scale;
            }
        } else {  // model/gaussian.metal:76-135
            const float* act = static_cast<const float*>(actions) + (size_t)r * A;
            float logp = 0.0f;
            for (uint32_t k = 0; k < A; ++k) {
                float ls = logStd[k];
                float dd = (act[k] - h[k]) * mg::expf(-ls);
                logp += -0.5f * dd * dd - ls - kLogSqrt2Pi;
                entropy += ls + kLogSqrt2Pi + 0.5f;
            }
            logpA = logp;
            ratio = mg::expf(logp - old_logp[r]);
            float surr1 = ratio * a_n;
            float cr = std::min(std::max(ratio, 1.0f - hp->clip), 1.0f + hp->clip);
            float surr2 = cr * a_n;
            policyLoss = -std::min(surr1, surr2);
            gLogp = (surr1 <= surr2) ? -a_n * ratio : 0.0f;
            for (uint32_t k = 0; k < A; ++k) {
                float ls = logStd[k];
                float invStd = mg::expf(-ls);
                float dd = (act[k] - h[k]) * invStd;
                dz[k] = gLogp * dd * invStd * scale;
                dls[(size_t)r * A + k] = (gLogp * (dd * dd - 1.0f) - hp->entropy_coef) * scale;
            }
        }
        float vErr = h[A] - ret[r];
        dz[A] = hp->value_coef * vErr * scale;
        float* st = &rowStats[(size_t)r * 5];
        st[0] = policyLoss;
        st[1] = 0.5f * hp->value_coef * vErr * vErr;
        st[2] = entropy;
        st[3] = old_logp[r] - logpA;
        st[4] = (std::fabs(ratio - 1.0f) > hp->clip) ? 1.0f : 0.0f;
    }

    // backward dX chain per row (model/ppo.h:793-865)
    std::vector<float> dxl((size_t)B * actW);     // gradient at each LN output
    std::vector<float> dhb((size_t)B * NL * E);   // gradient at each block output (dStream)
    std::vector<float> dvb((size_t)B * NL * H);   // masked dV per block
    std::vector<float> dh0((size_t)B * E);        // gradient at the embed output
    parallel_for(B, threads, [&](uint32_t b, uint32_t e) {
        std::vector<float> dx(E), dh(E), dv(H), tmp(E);
        for (uint32_t r = b; r < e; ++r) {
            const float* dz = &dhead[(size_t)r * HD];
            const float* Wh = P + L.off_head;
            for (uint32_t k = 0; k < E; ++k) {  // model/linear.metal:40-60
                float acc = 0.0f;
                for (uint32_t j = 0; j < HD; ++j) acc += dz[j] * Wh[k * HD + j];
                dx[k] = acc;
            }
            std::memcpy(&dxl[r * actW + NL * E], dx.data(), E * 4);
            ln_backward(dx.data(), &xn[r * actW + NL * E], P + L.off_ln_gamma[NL], sd[(size_t)r * (NL + 1) + NL], E,
                        dh.data());
            for (int l = (int)NL - 1; l >= 0; --l) {
                // bf16 mode: dh and dV enter their GEMMs (and the weight
                // gradients) rounded, and so do the weights
                const bool bf = d.bf16 != 0;
                auto q = [bf](float z) { return bf ? round_bf16(z) : z; };
                for (uint32_t c = 0; c < E; ++c) dhb[((size_t)r * NL + l) * E + c] = q(dh[c]);
                const float* dhq = &dhb[((size_t)r * NL + l) * E];
                const float* Dn = P + L.off_down[l];
                const float* Up = P + L.off_up[l];
                for (uint32_t j = 0; j < H; ++j) {  // model/mlp.metal:88-127
                    float acc = 0.0f;
                    const float* row = Dn + (size_t)j * E;
                    for (uint32_t c = 0; c < E; ++c) acc += dhq[c] * q(row[c]);
                    dv[j] = q(passes(r, (uint32_t)l, j) ? acc : 0.0f);
                }
                std::memcpy(&dvb[((size_t)r * NL + l) * H], dv.data(), H * 4);
                for (uint32_t k = 0; k < E; ++k) {  // model/mlp.metal:131-153
                    float acc = 0.0f;
                    const float* row = Up + (size_t)k * H;
                    for (uint32_t j = 0; j < H; ++j) acc += dv[j] * q(row[j]);
                    dx[k] = acc;
                }
                std::memcpy(&dxl[r * actW + (size_t)l * E], dx.data(), E * 4);
                ln_backward(dx.data(), &xn[r * actW + (size_t)l * E], P + L.off_ln_gamma[l],
                            sd[(size_t)r * (NL + 1) + l], E, tmp.data());
                for (uint32_t c = 0; c < E; ++c) dh[c] = tmp[c] + dh[c];  // residualAdd(dBranch, dStream)
            }
            std::memcpy(&dh0[(size_t)r * E], dh.data(), E * 4);
        }
    });

    // weight gradients: sums over rows in row order
    std::vector<float> g(L.count, 0.0f);
    auto reduce = [&](uint32_t nOut, uint32_t off, auto term) {
        parallel_for(nOut, threads, [&](uint32_t b, uint32_t e) {
            for (uint32_t o = b; o < e; ++o) {
                float acc = 0.0f;
                for (uint32_t r = 0; r < B; ++r) acc += term(r, o);
                g[off + o] = acc;
            }
        });
    };
    // model/input.metal:38-60
    reduce(O * E, L.off_in_w, [&](uint32_t r, uint32_t o) { return obs[(size_t)r * O + o / E] * dh0[(size_t)r * E + o % E]; });
    reduce(E, L.off_in_b, [&](uint32_t r, uint32_t o) { return dh0[(size_t)r * E + o]; });
    // model/layernorm.metal:80-81 (dgamma += xn dZ, dbeta += dZ)
    for (uint32_t l = 0; l <= NL; ++l) {
        reduce(E, L.off_ln_gamma[l], [&](uint32_t r, uint32_t o) {
            return xn[r * actW + (size_t)l * E + o] * dxl[r * actW + (size_t)l * E + o];
        });
        reduce(E, L.off_ln_beta[l], [&](uint32_t r, uint32_t o) { return dxl[r * actW + (size_t)l * E + o]; });
    }
    for (uint32_t l = 0; l < NL; ++l) {  // model/mlp.metal:167-208
        reduce(E * H, L.off_up[l], [&](uint32_t r, uint32_t o) {
            return x[r * actW + (size_t)l * E + o / H] * dvb[((size_t)r * NL + l) * H + o % H];
        });
        reduce(H * E, L.off_down[l], [&](uint32_t r, uint32_t o) {
            return vv[((size_t)r * NL + l) * H + o / E] * dhb[((size_t)r * NL + l) * E + o % E];
        });
    }
    // model/linear.metal:71-93
    reduce(E * HD, L.off_head, [&](uint32_t r, uint32_t o) {
        return x[r * actW + (size_t)NL * E + o / HD] * dhead[(size_t)r * HD + o % HD];
    });
    if (d.continuous)  // model/gaussian.metal:166-168
        reduce(A, L.off_log_std, [&](uint32_t r, uint32_t o) { return dls[(size_t)r * A + o]; });
    if (grad_out) std::memcpy(grad_out, g.data(), (size_t)L.count * 4);

    // model/optimizer.metal:23-60 with the host step of model/ppo.h:873-881
    // The reference adds per-SIMD partial squares with float atomics in an
    // unspecified order; the checker accumulates in double, then rounds once.
    double normSqD = 0.0;
    for (uint32_t i = 0; i < L.count; ++i) normSqD += (double)g[i] * (double)g[i];
    float normSq = (float)normSqD;
    const float beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
    float b1p = std::pow(beta1, (float)step), b2p = std::pow(beta2, (float)step);
    float norm = std::sqrt(normSq);
    float clipScale = (hp->max_grad_norm > 0.0f && norm > hp->max_grad_norm) ? hp->max_grad_norm / (norm + 1e-6f) : 1.0f;
    for (uint32_t i = 0; i < L.count; ++i) {
        float gi = g[i] * clipScale;
        float m = beta1 * M[i] + (1.0f - beta1) * gi;
        float v = beta2 * V[i] + (1.0f - beta2) * gi * gi;
        M[i] = m;
        V[i] = v;
        float mHat = m / (1.0f - b1p);
        float vHat = v / (1.0f - b2p);
        P[i] = P[i] - hp->lr * mHat / (std::sqrt(vHat) + eps);
    }

    // model/ppo.h:925-943
    orc_stats st{0, 0, 0, 0, 0, 0};
    for (uint32_t r = 0; r < B; ++r) {
        st.policy += rowStats[r * 5 + 0];
        st.value += rowStats[r * 5 + 1];
        st.entropy += rowStats[r * 5 + 2];
        st.approx_kl += rowStats[r * 5 + 3];
        st.clip_frac += rowStats[r * 5 + 4];
    }
    float invB = 1.0f / (float)B;
    st.policy *= invB;
    st.value *= invB;
    st.entropy *= invB;
    st.approx_kl *= invB;
    st.clip_frac *= invB;
    st.grad_norm = norm;
    if (stats) *stats = st;
}

void orc_shuffle_state_init(uint32_t seed, uint64_t* state) { *state = kShuffleStream ^ (uint64_t)seed; }

// Fisher-Yates over the current order, in place (std::shuffle's role at model/ppo.h:920)
void orc_shuffle_blocks(uint64_t* state, uint32_t* order, uint32_t count) {
    for (uint32_t i = count; i > 1; --i) {
        uint32_t j = (uint32_t)(splitmix(*state) % (uint64_t)i);
        std::swap(order[i - 1], order[j]);
    }
}

void orc_train(const orc_dims* d, const orc_hparams* hp, float* params, float* m, float* v, uint32_t* step,
               uint64_t* shuffle_state, uint32_t n, uint32_t horizon, uint32_t minibatch, uint32_t epochs,
               const float* obs_slots, const void* action_slots, const float* adv_slots, const float* ret_slots,
               const float* logp_slots, orc_stats* stats_out, uint32_t* order_inout, int threads) {
    const uint32_t perSlot = n / minibatch, blocks = horizon * perSlot;
    const uint32_t O = d->obs_dim;
    const size_t ab = d->continuous ? (size_t)d->act_dim * 4 : 4;
    uint32_t mb = 0;
    for (uint32_t e = 0; e < epochs; ++e) {
        orc_shuffle_blocks(shuffle_state, order_inout, blocks);
        for (uint32_t k = 0; k < blocks; ++k) {
            uint32_t blk = order_inout[k];
            uint32_t t = blk / perSlot, r0 = (blk % perSlot) * minibatch;
            size_t row = (size_t)t * n + r0;
            *step += 1;
            orc_train_minibatch(d, hp, params, m, v, *step, minibatch, obs_slots + row * O,
                                static_cast<const char*>(action_slots) + row * ab, adv_slots + row, ret_slots + row,
                                logp_slots + row, nullptr, stats_out ? &stats_out[mb] : nullptr, nullptr, threads);
            ++mb;
        }
    }
}

}  // extern "C"
