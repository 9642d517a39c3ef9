// The fast-mode dK/dV kernel for head dims up to 64, in a translation unit of
// its own: the build compiles it with every MFMA in its vector-register form
// (-mllvm -amdgpu-mfma-vgpr-form).  Then the S and dP products land in the
// registers their softmax reads, instead of in accumulation registers that
// each element is first copied out of (128 copies per 128-query step).  At
// these head dims everything still fits the register file; at D = 128 it does
// not (attn_bwd_fast.hip keeps that instantiation in the default form).
#include "attn_bwd_dkdv_fast.hpp"

namespace fc {

hipError_t launch_bwd_dkdv_fast_vgpr(const Problem& p, const BwdArgs& a, hipStream_t s) {
  switch (p.Dk) {
    case 16: return launch_dkdv_fast_t<16>(p, a, s);
    case 32: return launch_dkdv_fast_t<32>(p, a, s);
    case 64: return launch_dkdv_fast_t<64>(p, a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fc
