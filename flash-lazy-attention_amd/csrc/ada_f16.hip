// AdaSplash forward / backward instantiations for F16 inputs.
#include "ada_fwd.inc"
#include "ada_bwd.inc"

namespace fla {
template hipError_t ada_fwd_launch<F16, 32>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_fwd_launch<F16, 64>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_fwd_launch<F16, 128>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<F16, 32>(const AdaBwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<F16, 64>(const AdaBwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<F16, 128>(const AdaBwdArgs&, int, hipStream_t);
}  // namespace fla
