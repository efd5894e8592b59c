// Backward RMSNorm kernel instantiations with 3 chunk(s) per lane.
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace rms {

BwdKernel bwd_kernel_vpl3(int wpr, int nx, int ndy, bool res, bool fwd) {
  switch (wpr) {
    case 1: return bwd_for_terms<3, 1>(nx, ndy, res, fwd);
    case 2: return bwd_for_terms<3, 2>(nx, ndy, res, fwd);
    case 4: return bwd_for_terms<3, 4>(nx, ndy, res, fwd);
  }
  return nullptr;
}

}  // namespace rms
}  // namespace kp
