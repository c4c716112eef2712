// Deterministic float math shared by host and device code.
//
// Environment dynamics and samplers must give the same bits on the CPU and on
// the GPU: one ulp of difference in sin(theta) near CartPole's 12-degree
// threshold flips a done flag, and a flipped done flag changes how many reset
// draws an env takes from its RNG stream. libm and the device libraries do not
// promise identical results, so every transcendental used by per-env code is
// computed here from IEEE float arithmetic only (+, -, *, / and exact bit
// manipulation), in one fixed order. IEEE float operations are correctly
// rounded on x86-64 SSE and on CDNA, so both sides agree bit for bit as long as
// floating-point contraction is off (every build of this project passes
// -ffp-contract=off). Tested against correctly rounded values: expf, sinf and
// cosf within 1 ulp, logf within 2, tanhf within 3. sin/cos arguments with
// |x| >= 8 take an exact double-precision path, identically on both sides.
//
// Methods (all textbook, named per function):
//   expf   : x = k ln2 + r (Cody & Waite 1980, two-part ln2 whose high part
//            has 9 significant bits, so k * high is exact), Taylor series of
//            e^r to degree 7, scaled by 2^k through the exponent bits.
//   logf   : x = 2^e m, m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(s),
//            s = (m-1)/(m+1), odd series to s^9 (Abramowitz & Stegun 4.1.27).
//   sincosf: reduction by pi/2 with a three-part pi/2 (Cody & Waite), Taylor
//            series on [-pi/4, pi/4] to degree 9 (sin) and 10 (cos),
//            quadrant selection; |x| <= pi/4 skips the reduction.
//   tanhf  : tanh |x| = expm1(2|x|) / (expm1(2|x|) + 2), expm1 by its Taylor
//            series below 0.5, else e^y - 1.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define MG_HD __host__ __device__ inline
#else
#define MG_HD inline
#endif

namespace mg {

MG_HD uint32_t float_to_bits(float f) {
    union { float f; uint32_t u; } v;
    v.f = f;
    return v.u;
}
MG_HD float bits_to_float(uint32_t b) {
    union { uint32_t u; float f; } v;
    v.u = b;
    return v.f;
}

// Round-half-away-from-zero to an integer, for arguments well inside int range.
MG_HD int round_to_int(double x) { return x >= 0.0 ? (int)(x + 0.5) : -(int)(-x + 0.5); }

constexpr double kTwoOverPi = 6.36619772367581382433e-01;
constexpr double kPio2_1 = 1.57079632673412561417e+00;   // first 33 bits of pi/2
constexpr double kPio2_2 = 6.07710050630396597660e-11;   // next 33 bits
constexpr double kPio2_3 = 2.02226624879595063154e-21;   // remainder

MG_HD double sin_taylor_d(double r) {  // |r| <= pi/4, degree 17
    double r2 = r * r;
    double q = 1.0 / 355687428096000.0;   // 1/17!
    q = q * r2 - 1.0 / 1307674368000.0;   // 1/15!
    q = q * r2 + 1.0 / 6227020800.0;      // 1/13!
    q = q * r2 - 1.0 / 39916800.0;        // 1/11!
    q = q * r2 + 1.0 / 362880.0;          // 1/9!
    q = q * r2 - 1.0 / 5040.0;            // 1/7!
    q = q * r2 + 1.0 / 120.0;             // 1/5!
    q = q * r2 - 1.0 / 6.0;               // 1/3!
    return r + r * r2 * q;
}

MG_HD double cos_taylor_d(double r) {  // |r| <= pi/4, degree 18
    double r2 = r * r;
    double q = -1.0 / 6402373705728000.0;  // -1/18!
    q = q * r2 + 1.0 / 20922789888000.0;   // 1/16!
    q = q * r2 - 1.0 / 87178291200.0;      // 1/14!
    q = q * r2 + 1.0 / 479001600.0;        // 1/12!
    q = q * r2 - 1.0 / 3628800.0;          // 1/10!
    q = q * r2 + 1.0 / 40320.0;            // 1/8!
    q = q * r2 - 1.0 / 720.0;              // 1/6!
    q = q * r2 + 1.0 / 24.0;               // 1/4!
    q = q * r2 - 0.5;                      // 1/2!
    return 1.0 + r2 * q;
}

// Reduce x by multiples of pi/2: returns r in about [-pi/4, pi/4], quadrant in *q.
// Accurate for |x| < 2^19 * pi/2, far beyond what env dynamics feed it.
MG_HD double reduce_pio2(float x, int* q) {
    double xd = (double)x;
    int k = round_to_int(xd * kTwoOverPi);
    double kd = (double)k;
    double r = ((xd - kd * kPio2_1) - kd * kPio2_2) - kd * kPio2_3;
    *q = k & 3;
    return r;
}

// ---- float paths ------------------------------------------------------------

// 2^k as a float for k in [-126, 127], exact.
MG_HD float pow2_f(int k) { return bits_to_float((uint32_t)(k + 127) << 23); }

// Round to nearest integer (ties away from zero) for |x| < 2^22.
MG_HD int round_to_int_f(float x) { return x >= 0.0f ? (int)(x + 0.5f) : -(int)(-x + 0.5f); }

constexpr float kLn2HiF = 0.693359375f;         // 355/512: k * kLn2HiF is exact for |k| < 2^15
constexpr float kLn2LoF = -2.12194440e-4f;      // ln2 - kLn2HiF
constexpr float kInvLn2F = 1.44269502162933349609f;

// e^r for |r| <= 0.35 by Taylor series (Horner), degree 7.
MG_HD float exp_taylor_f(float r) {
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return p;
}

// e^x. Arguments below -87 return 0, so every nonzero result is a normal
// float (no dependence on either side's subnormal handling).
MG_HD float expf(float x) {
    if (x != x) return x;
    if (x > 88.7228394f) return bits_to_float(0x7f800000u);
    if (x < -87.0f) return 0.0f;
    const int k = round_to_int_f(x * kInvLn2F);
    const float kf = (float)k;
    const float r = (x - kf * kLn2HiF) - kf * kLn2LoF;
    const float p = exp_taylor_f(r);
    // two factors so each stays a normal float at the ends of the range
    const int k1 = k / 2;
    return (p * pow2_f(k1)) * pow2_f(k - k1);
}

// e^y - 1 for y >= 0.
MG_HD float expm1_pos_f(float y) {
    if (y < 0.5f) {
        float p = 1.0f / 40320.0f;  // 1/8!
        p = p * y + 1.0f / 5040.0f;
        p = p * y + 1.0f / 720.0f;
        p = p * y + 1.0f / 120.0f;
        p = p * y + 1.0f / 24.0f;
        p = p * y + 1.0f / 6.0f;
        p = p * y + 0.5f;
        p = p * y + 1.0f;
        return p * y;
    }
    return expf(y) - 1.0f;
}

MG_HD float tanhf(float x) {
    if (x != x) return x;
    const float ax = x < 0.0f ? -x : x;
    if (ax > 9.0f) return x < 0.0f ? -1.0f : 1.0f;
    const float e = expm1_pos_f(2.0f * ax);
    const float t = e / (e + 2.0f);
    return x < 0.0f ? -t : t;
}

MG_HD float logf(float x) {
    uint32_t b = float_to_bits(x);
    if (x != x) return x;
    if (x < 0.0f) return bits_to_float(0x7fc00000u);
    if (x == 0.0f) return bits_to_float(0xff800000u);
    if (b == 0x7f800000u) return x;
    int e = 0;
    if ((b >> 23) == 0) {  // subnormal: scale by 2^25
        x = x * 33554432.0f;
        b = float_to_bits(x);
        e = -25;
    }
    e += (int)(b >> 23) - 127;
    float m = bits_to_float((b & 0x007fffffu) | 0x3f800000u);  // [1, 2)
    if (m > 1.41421356f) {
        m = m * 0.5f;
        e += 1;
    }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 1.0f / 9.0f;
    p = p * s2 + 1.0f / 7.0f;
    p = p * s2 + 1.0f / 5.0f;
    p = p * s2 + 1.0f / 3.0f;
    const float ef = (float)e;
    // log x = e ln2 + 2 s + 2 s^3 p, small terms first
    const float lm = 2.0f * s + (2.0f * s) * s2 * p;
    return ef * kLn2HiF + (ef * kLn2LoF + lm);
}

MG_HD float sin_taylor_f(float r) {  // |r| <= pi/4, degree 9
    const float r2 = r * r;
    float q = 1.0f / 362880.0f;
    q = q * r2 - 1.0f / 5040.0f;
    q = q * r2 + 1.0f / 120.0f;
    q = q * r2 - 1.0f / 6.0f;
    return r + r * r2 * q;
}

MG_HD float cos_taylor_f(float r) {  // |r| <= pi/4, degree 10
    const float r2 = r * r;
    float q = -1.0f / 3628800.0f;
    q = q * r2 + 1.0f / 40320.0f;
    q = q * r2 - 1.0f / 720.0f;
    q = q * r2 + 1.0f / 24.0f;
    q = q * r2 - 0.5f;
    return 1.0f + r2 * q;
}

constexpr float kPio4F = 0.785398163f;
constexpr float kTwoOverPiF = 0.636619746685028076171875f;
// pi/2 = kPio2_1F + kPio2_2F + kPio2_3F: the first two have 8 and 12
// significant bits (k times either is exact for the |k| <= 5 of the float
// path), the third is the float nearest the remainder.
constexpr float kPio2_1F = 1.5703125f;
constexpr float kPio2_2F = 4.83870506286621093750e-4f;
constexpr float kPio2_3F = -4.37113883e-8f;

// sin and cos of x with one shared reduction.
MG_HD void sincosf(float x, float* s, float* c) {
    if (x != x || float_to_bits(x) << 1 == 0xff000000u) {  // NaN, +-inf
        *s = *c = bits_to_float(0x7fc00000u);
        return;
    }
    const float ax = x < 0.0f ? -x : x;
    if (ax <= kPio4F) {
        *s = sin_taylor_f(x);
        *c = cos_taylor_f(x);
        return;
    }
    float r;
    int q;
    if (ax < 8.0f) {
        const int k = round_to_int_f(x * kTwoOverPiF);
        const float kf = (float)k;
        r = ((x - kf * kPio2_1F) - kf * kPio2_2F) - kf * kPio2_3F;
        q = k & 3;
        const float sr = sin_taylor_f(r), cr = cos_taylor_f(r);
        switch (q) {
            case 0: *s = sr, *c = cr; break;
            case 1: *s = cr, *c = -sr; break;
            case 2: *s = -sr, *c = -cr; break;
            default: *s = -cr, *c = sr; break;
        }
        return;
    }
    // large arguments: the exact double-precision path
    const double rd = reduce_pio2(x, &q);
    const double sd = sin_taylor_d(rd), cd = cos_taylor_d(rd);
    switch (q) {
        case 0: *s = (float)sd, *c = (float)cd; break;
        case 1: *s = (float)cd, *c = (float)-sd; break;
        case 2: *s = (float)-sd, *c = (float)-cd; break;
        default: *s = (float)-cd, *c = (float)sd; break;
    }
}

MG_HD float sinf(float x) {
    float s, c;
    sincosf(x, &s, &c);
    return s;
}

MG_HD float cosf(float x) {
    float s, c;
    sincosf(x, &s, &c);
    return c;
}

}  // namespace mg
