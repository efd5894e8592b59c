// Backward RMSNorm kernel instantiations with 2 chunk(s) per lane.
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace rms {

BwdKernel bwd_kernel_vpl2(int wpr, int nx, int ndy, bool res, bool fwd) {
  switch (wpr) {
    case 1: return bwd_for_terms<2, 1>(nx, ndy, res, fwd);
    case 2: return bwd_for_terms<2, 2>(nx, ndy, res, fwd);
    case 4: return bwd_for_terms<2, 4>(nx, ndy, res, fwd);
    case 8: return bwd_for_terms<2, 8, 8>(nx, ndy, res, fwd);  // N = 8192: 8-wave blocks, one row per step
  }
  return nullptr;
}

}  // namespace rms
}  // namespace kp
