// Forward RMSNorm kernel instantiations (every fast-path row shape).
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace rms {

FwdKernel fwd_kernel(int vpl, int wpr, int nx) {
  switch (vpl * 10 + wpr) {
    case 11: return fwd_for_terms<1, 1>(nx);
    case 21: return fwd_for_terms<2, 1>(nx);
    case 31: return fwd_for_terms<3, 1>(nx);
    case 41: return fwd_for_terms<4, 1>(nx);
    case 51: return fwd_for_terms<5, 1>(nx);
    case 12: return fwd_for_terms<1, 2>(nx);
    case 22: return fwd_for_terms<2, 2>(nx);
    case 32: return fwd_for_terms<3, 2>(nx);
    case 42: return fwd_for_terms<4, 2>(nx);
    case 52: return fwd_for_terms<5, 2>(nx);
    case 14: return fwd_for_terms<1, 4>(nx);
    case 24: return fwd_for_terms<2, 4>(nx);
    case 34: return fwd_for_terms<3, 4>(nx);
    case 44: return fwd_for_terms<4, 4>(nx);
    case 61: return fwd_for_terms<6, 1>(nx);
    case 81: return fwd_for_terms<8, 1>(nx);
    case 82: return fwd_for_terms<8, 2>(nx);
  }
  return nullptr;
}

}  // namespace rms
}  // namespace kp
