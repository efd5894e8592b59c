// Backward RMSNorm kernel instantiations with 5 chunks per lane.
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace rms {

BwdKernel bwd_kernel_vpl5(int wpr, int nx, int ndy, bool res, bool fwd) {
  switch (wpr) {
    case 1: return bwd_for_terms<5, 1>(nx, ndy, res, fwd);
    case 2: return bwd_for_terms<5, 2>(nx, ndy, res, fwd);
  }
  return nullptr;
}

// 6 and 8 chunks per lane (reached only through the KP_RMS_VPL_MAX tuning knob).
BwdKernel bwd_kernel_vpl68(int vpl, int wpr, int nx, int ndy, bool res, bool fwd) {
  switch (vpl * 10 + wpr) {
    case 61: return bwd_for_terms<6, 1>(nx, ndy, res, fwd);
    case 81: return bwd_for_terms<8, 1>(nx, ndy, res, fwd);
    case 82: return bwd_for_terms<8, 2>(nx, ndy, res, fwd);
  }
  return nullptr;
}

}  // namespace rms
}  // namespace kp
