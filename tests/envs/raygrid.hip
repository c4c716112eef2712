// Instantiates and registers the test-only ray-casting envs (see raygrid.h:
// RayGrid, RayField and their split twins) in the test env library.
#include "mg/device/env_kernels.h"
#include "raygrid.h"

MG_DEFINE_ENV(RayGrid)
MG_DEFINE_ENV(RayGridSplit)
MG_DEFINE_ENV(RayField)
MG_DEFINE_ENV(RayFieldSplit)
