// AdaSplash forward / backward instantiations for F32 inputs.
#include "ada_fwd.inc"
#include "ada_bwd.inc"

namespace fla {
template hipError_t ada_fwd_launch<F32, 32>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_fwd_launch<F32, 64>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_fwd_launch<F32, 128>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<F32, 32>(const AdaBwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<F32, 64>(const AdaBwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<F32, 128>(const AdaBwdArgs&, int, hipStream_t);
}  // namespace fla
