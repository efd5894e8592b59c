// Forward RMSNorm kernel instantiations with the embedding gather fused in
// (one term whose rows are picked by token ids), every fast-path row shape.
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace rms {

FwdKernel fwd_gather_kernel(int vpl, int wpr) {
  switch (vpl * 10 + wpr) {
    case 11: return rms_fwd_vec<1, 1, 1, true>;
    case 21: return rms_fwd_vec<2, 1, 1, true>;
    case 31: return rms_fwd_vec<3, 1, 1, true>;
    case 41: return rms_fwd_vec<4, 1, 1, true>;
    case 51: return rms_fwd_vec<5, 1, 1, true>;
    case 12: return rms_fwd_vec<1, 2, 1, true>;
    case 22: return rms_fwd_vec<2, 2, 1, true>;
    case 32: return rms_fwd_vec<3, 2, 1, true>;
    case 42: return rms_fwd_vec<4, 2, 1, true>;
    case 52: return rms_fwd_vec<5, 2, 1, true>;
    case 14: return rms_fwd_vec<1, 4, 1, true>;
    case 24: return rms_fwd_vec<2, 4, 1, true>;
    case 34: return rms_fwd_vec<3, 4, 1, true>;
    case 44: return rms_fwd_vec<4, 4, 1, true>;
    case 61: return rms_fwd_vec<6, 1, 1, true>;
    case 81: return rms_fwd_vec<8, 1, 1, true>;
    case 82: return rms_fwd_vec<8, 2, 1, true>;
  }
  return nullptr;
}

}  // namespace rms
}  // namespace kp
