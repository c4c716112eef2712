// Built-in envs: CartPoleContinuous with the tanh force, and the reference's
// clamped-force variant (examples/CartPoleContinuous/cartpole_continuous.metal:81-90).
#include "mg/device/env_kernels.h"
#include "mg/envs/cartpole_continuous.h"

MG_DEFINE_ENV(CartPoleContinuous)
MG_DEFINE_ENV(CartPoleContinuousClamp)
