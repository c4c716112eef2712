// Instantiates and registers the Corridor env's kernels (compiled with hipcc).
#include "mg/device/env_kernels.h"
#include "corridor.h"

MG_DEFINE_ENV(Corridor)
