// Instantiating an env's kernels: the MI355X counterpart of the reference's
//   template [[host_name("rollout_x")]] kernel void rollout<X>(...);
// line (README.md:42-52). In a .hip file compiled with hipcc:
//
//   #include <mg/device/env_kernels.h>
//   #include "my_env.h"
//   MG_DEFINE_ENV(MyEnv)
//
// This instantiates rollout<MyEnv> and collect<MyEnv> and registers them with
// libmetalgym_amd under MyEnv::KERNEL at load time, where Gym<MyEnv> finds
// them (gym.h:43-44). `MyEnv` must be a plain identifier.
#pragma once
#include "collect.h"
#include "rollout.h"

namespace mg {
namespace dev {

template <typename Env>
mg_env_desc make_env_desc() {
    using Tr = EnvTraits<Env>;
    mg_env_desc d{};
    d.abi_version = MG_ABI_VERSION;
    d.state_bytes = (uint32_t)sizeof(typename Env::State);
    d.action_bytes = (uint32_t)sizeof(typename Env::Action);
    d.obs_dim = Env::OBS_DIM;
    d.act_dim = Env::ACT_DIM;
    d.continuous = Tr::CONTINUOUS ? 1u : 0u;
    d.state_in_registers = Tr::STATE_IN_REGISTERS ? 1u : 0u;
    d.kernel = Env::KERNEL;
    d.rollout = &launch_rollout<Env>;
    d.collect = &launch_collect<Env>;
    return d;
}

}  // namespace dev
}  // namespace mg

#define MG_DEFINE_ENV(Env)                                                          \
    namespace {                                                                     \
    const mg_env_desc mg_env_desc_##Env = ::mg::dev::make_env_desc<Env>();          \
    const int mg_env_registered_##Env = mg_env_register(&mg_env_desc_##Env);        \
    }
