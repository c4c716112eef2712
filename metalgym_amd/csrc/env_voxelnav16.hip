// Built-in env: VoxelNav16, the gather-heavy 16^3 voxel navigation env.
#include "mg/device/env_kernels.h"
#include "mg/envs/voxelnav16.h"

MG_DEFINE_ENV(VoxelNav16)
