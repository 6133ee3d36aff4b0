// Lazy attention forward / backward instantiations for F16 inputs.
#include "lazy.inc"

namespace fla {
template hipError_t lazy_fwd_launch<F16, 32>(const LazyArgs&, hipStream_t);
template hipError_t lazy_fwd_launch<F16, 64>(const LazyArgs&, hipStream_t);
template hipError_t lazy_fwd_launch<F16, 128>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<F16, 32>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<F16, 64>(const LazyArgs&, hipStream_t);
template hipError_t lazy_bwd_launch<F16, 128>(const LazyArgs&, hipStream_t);
}  // namespace fla
