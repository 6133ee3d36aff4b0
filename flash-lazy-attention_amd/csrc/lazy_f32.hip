// Lazy attention forward / backward instantiations for F32 inputs.
#include "lazy.inc"

namespace fla {
template hipError_t lazy_fwd_launch<F32, 32>(const LazyArgs&, hipStream_t);
template hipError_t lazy_fwd_launch<F32, 64>(const LazyArgs&, hipStream_t);
template hipError_t lazy_fwd_launch<F32, 128>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<F32, 32>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<F32, 64>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<F32, 128>(const LazyArgs&, hipStream_t);
}  // namespace fla
