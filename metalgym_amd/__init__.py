"""metalgym_amd: MetalGym's rollout-and-policy hot path on one AMD MI355X.

The product is the C ABI library ``metalgym_amd/lib/libmetalgym_amd.so``
(declared in ``include/mg/capi.h``) and the header-only C++ API on top of it
(``include/mg/gym.h``, ``include/mg/ppo.h``). This Python module is a thin
ctypes binding of that C ABI for tests and benchmarks. There is no fallback:
if the library has not been built, importing ``lib()`` raises.
"""
from ._capi import (  # noqa: F401
    LIB_PATH,
    COLLECT_FN,
    CapiError,
    CollectArgs,
    Gym,
    KernelTimes,
    LossStats,
    PPOConfig,
    PPOHParams,
    PPOModel,
    PolicyView,
    DeviceBuffer,
    build,
    d2h,
    env_desc,
    env_names,
    h2d,
    lib,
    timing_enable,
    timing_get,
    timing_reset,
    K_NAMES,
)
