// Built-in env: CartPole (examples/CartPole/cartpole.metal:78-87 instantiates
// rollout<CartPole> as "rollout_cartpole").
#include "mg/device/env_kernels.h"
#include "mg/envs/cartpole.h"

MG_DEFINE_ENV(CartPole)
