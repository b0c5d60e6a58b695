// stub_launch.cpp -- host-only stand-ins for the kernel launchers and the per-launch timing of
// libtda_hip.so, so that tda_host.cpp (the C ABI: validation, buffer sizing, parameter set-up)
// builds and runs with -fsanitize=address,undefined on a machine without a GPU.  Each launcher
// records the parameter block it was given; the driver (abi_driver.cpp) checks them.
#include <cstring>

#include "../../tda_amd/csrc/tda_params.hpp"
#include "stub_launch.hpp"

namespace stub {
int fwd_calls = 0, bwd_calls = 0;
tda::FwdParams last_fwd;
tda::BwdParams last_bwd;
tda::KernelKey last_key;
int fail_with = 0;  // a hipError_t value the next launch reports (0: success)
}  // namespace stub

namespace tda {
int launch_fwd(const FwdParams& p, const KernelKey& k, void*) {
  ++stub::fwd_calls;
  std::memcpy(&stub::last_fwd, &p, sizeof(p));
  stub::last_key = k;
  const int e = stub::fail_with;
  stub::fail_with = 0;
  return e;
}
int launch_bwd(const BwdParams& p, const KernelKey& k, void*) {
  ++stub::bwd_calls;
  std::memcpy(&stub::last_bwd, &p, sizeof(p));
  stub::last_key = k;
  const int e = stub::fail_with;
  stub::fail_with = 0;
  return e;
}
void timing_begin(void*) {}
void launched(void*, const char*) {}
int timing_end() { return 0; }
}  // namespace tda
