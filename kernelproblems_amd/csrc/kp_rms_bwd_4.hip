// Backward RMSNorm kernel instantiations with 4 chunk(s) per lane.
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace rms {

BwdKernel bwd_kernel_vpl4(int wpr, int nx, int ndy, bool res, bool fwd) {
  switch (wpr) {
    case 1: return bwd_for_terms<4, 1>(nx, ndy, res, fwd);
    case 2: return bwd_for_terms<4, 2>(nx, ndy, res, fwd);
    case 4: return bwd_for_terms<4, 4>(nx, ndy, res, fwd);
  }
  return nullptr;
}

}  // namespace rms
}  // namespace kp
