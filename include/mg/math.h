// Deterministic float math shared by host and device code.
//
// Environment dynamics and samplers must give the same bits on the CPU and on
// the GPU: one ulp of difference in sin(theta) near CartPole's 12-degree
// threshold flips a done flag, and a flipped done flag changes how many reset
// draws an env takes from its RNG stream. libm and the device libraries do not
// promise identical results, so every transcendental used by per-env code is
// computed here from IEEE double arithmetic only (+, -, *, / and exact bit
// manipulation), then rounded once to float. IEEE double operations are
// correctly rounded on x86-64 SSE2 and on CDNA, so both sides agree bit for bit
// as long as floating-point contraction is off (every build of this project
// passes -ffp-contract=off).
//
// Methods (all textbook, named per function):
//   expf   : argument reduction x = k ln2 + r (Cody & Waite 1980, two-part ln2),
//            Taylor series of e^r to degree 13, scaled by 2^k.
//   expm1  : Taylor series for |y| < 0.5, else exp - 1.
//   logf   : x = 2^e m, m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(s),
//            s = (m-1)/(m+1), odd series to s^21 (Abramowitz & Stegun 4.1.27).
//   sinf/cosf : reduction by pi/2 with a three-part pi/2 (Cody & Waite), Taylor
//            series on [-pi/4, pi/4] to degree 17/18, quadrant selection.
//   tanhf  : tanh x = expm1(2x) / (expm1(2x) + 2).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define MG_HD __host__ __device__ inline
#else
#define MG_HD inline
#endif

namespace mg {

MG_HD double bits_to_double(uint64_t b) {
    union { uint64_t u; double d; } v;
    v.u = b;
    return v.d;
}
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

// 2^k for k in [-1022, 1023], exact.
MG_HD double pow2_d(int k) { return bits_to_double((uint64_t)(k + 1023) << 52); }

// Round-half-away-from-zero to an integer, for arguments well inside int range.
MG_HD int round_to_int(double x) { return x >= 0.0 ? (int)(x + 0.5) : -(int)(-x + 0.5); }

constexpr double kLn2Hi = 6.93147180369123816490e-01;  // high part, exact in few bits
constexpr double kLn2Lo = 1.90821492927058770002e-10;  // ln2 - kLn2Hi
constexpr double kInvLn2 = 1.44269504088896338700e+00;
constexpr double kLn2 = 6.93147180559945286227e-01;

// e^r for |r| <= ln2/2 by Taylor series (Horner), degree 13.
MG_HD double exp_taylor_d(double r) {
    double p = 1.0 / 6227020800.0;  // 1/13!
    p = p * r + 1.0 / 479001600.0;  // 1/12!
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return p;
}

// e^x in double for |x| < 700.
MG_HD double exp_d(double x) {
    int k = round_to_int(x * kInvLn2);
    double r = (x - (double)k * kLn2Hi) - (double)k * kLn2Lo;
    return exp_taylor_d(r) * pow2_d(k);
}

MG_HD float expf(float x) {
    if (x != x) return x;
    if (x > 88.7228394f) return bits_to_float(0x7f800000u);
    if (x < -103.972084f) return 0.0f;
    double xd = (double)x;
    int k = round_to_int(xd * kInvLn2);
    double r = (xd - (double)k * kLn2Hi) - (double)k * kLn2Lo;
    double p = exp_taylor_d(r);
    // split the scale so each factor stays a normal double
    int k1 = k / 2;
    return (float)(p * pow2_d(k1) * pow2_d(k - k1));
}

// e^y - 1 in double.
MG_HD double expm1_d(double y) {
    if (y > -0.5 && y < 0.5) {
        // Taylor series y + y^2/2! + ... + y^18/18!
        double p = 1.0 / 6402373705728000.0;  // 1/18!
        p = p * y + 1.0 / 355687428096000.0;
        p = p * y + 1.0 / 20922789888000.0;
        p = p * y + 1.0 / 1307674368000.0;
        p = p * y + 1.0 / 87178291200.0;
        p = p * y + 1.0 / 6227020800.0;
        p = p * y + 1.0 / 479001600.0;
        p = p * y + 1.0 / 39916800.0;
        p = p * y + 1.0 / 3628800.0;
        p = p * y + 1.0 / 362880.0;
        p = p * y + 1.0 / 40320.0;
        p = p * y + 1.0 / 5040.0;
        p = p * y + 1.0 / 720.0;
        p = p * y + 1.0 / 120.0;
        p = p * y + 1.0 / 24.0;
        p = p * y + 1.0 / 6.0;
        p = p * y + 0.5;
        p = p * y + 1.0;
        return p * y;
    }
    return exp_d(y) - 1.0;
}

MG_HD float tanhf(float x) {
    if (x != x) return x;
    if (x > 10.0f) return 1.0f;
    if (x < -10.0f) return -1.0f;
    double e = expm1_d(2.0 * (double)x);
    return (float)(e / (e + 2.0));
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
    double m = (double)bits_to_float((b & 0x007fffffu) | 0x3f800000u);  // [1, 2)
    if (m > 1.41421356237309504880) {
        m = m * 0.5;
        e += 1;
    }
    double s = (m - 1.0) / (m + 1.0);
    double s2 = s * s;
    double p = 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    p = p * s2 + 1.0;
    double lm = 2.0 * s * p;
    return (float)((double)e * kLn2 + lm);
}

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

MG_HD float sinf(float x) {
    if (x != x) return x;
    if (float_to_bits(x) << 1 == 0xff000000u) return bits_to_float(0x7fc00000u);  // +-inf
    int q;
    double r = reduce_pio2(x, &q);
    double v;
    switch (q) {
        case 0: v = sin_taylor_d(r); break;
        case 1: v = cos_taylor_d(r); break;
        case 2: v = -sin_taylor_d(r); break;
        default: v = -cos_taylor_d(r); break;
    }
    return (float)v;
}

MG_HD float cosf(float x) {
    if (x != x) return x;
    if (float_to_bits(x) << 1 == 0xff000000u) return bits_to_float(0x7fc00000u);
    int q;
    double r = reduce_pio2(x, &q);
    double v;
    switch (q) {
        case 0: v = cos_taylor_d(r); break;
        case 1: v = -sin_taylor_d(r); break;
        case 2: v = -cos_taylor_d(r); break;
        default: v = sin_taylor_d(r); break;
    }
    return (float)v;
}

}  // namespace mg
