// Lazy attention forward / backward instantiations for BF16 inputs.
#include "lazy.inc"

namespace fla {
template hipError_t lazy_fwd_launch<BF16, 32>(const LazyArgs&, hipStream_t);
template hipError_t lazy_fwd_launch<BF16, 64>(const LazyArgs&, hipStream_t);
template hipError_t lazy_fwd_launch<BF16, 128>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<BF16, 32>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<BF16, 64>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<BF16, 128>(const LazyArgs&, hipStream_t);
}  // namespace fla
