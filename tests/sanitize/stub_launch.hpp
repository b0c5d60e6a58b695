// stub_launch.hpp -- what the stub launchers of stub_launch.cpp recorded.
#pragma once
#include "../../tda_amd/csrc/tda_params.hpp"

namespace stub {
extern int fwd_calls, bwd_calls;
extern tda::FwdParams last_fwd;
extern tda::BwdParams last_bwd;
extern tda::KernelKey last_key;
extern int fail_with;
}  // namespace stub
