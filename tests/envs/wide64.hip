// Instantiates and registers the test-only wide envs (see wide64.h). Loaded by
// the GPU tests as a separate library, the way a user's env library is.
#include "mg/device/env_kernels.h"
#include "wide64.h"

MG_DEFINE_ENV(Wide64)
MG_DEFINE_ENV(Wide64Gauss)
