// AdaSplash forward / backward instantiations for BF16 inputs.
#include "ada_fwd.inc"
#include "ada_bwd.inc"

namespace fla {
template hipError_t ada_fwd_launch<BF16, 32>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_fwd_launch<BF16, 64>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_fwd_launch<BF16, 128>(const AdaFwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<BF16, 32>(const AdaBwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<BF16, 64>(const AdaBwdArgs&, int, hipStream_t);
template hipError_t ada_bwd_launch<BF16, 128>(const AdaBwdArgs&, int, hipStream_t);
}  // namespace fla
