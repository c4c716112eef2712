// bfloat16 values as their 16-bit patterns (the upper half of an IEEE float),
// for host and device code alike.
#pragma once
#include <stdint.h>
#include <string.h>

#include "math.h"

namespace mg {

// Round to nearest, ties to even (the rounding of v_cvt_pk_bf16_f32 and of the
// usual float -> bfloat16 conversions) for finite x: add 0x7FFF plus the
// lowest kept bit, then truncate.
MG_HD uint16_t bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

MG_HD float bf16_to_float(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float x;
    memcpy(&x, &u, 4);
    return x;
}

}  // namespace mg
