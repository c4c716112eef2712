// Built-in env: VoxelNav, the reference's heightmap navigation env.
#include "mg/device/env_kernels.h"
#include "mg/envs/voxelnav.h"

MG_DEFINE_ENV(VoxelNav)
