// Lazy attention KV-cache (decode) forward instantiations for F32 inputs.
#include "lazy_decode.inc"

namespace fla {
template hipError_t lazy_decode_launch<F32, 32>(const LazyDecArgs&, hipStream_t);
template hipError_t lazy_decode_launch<F32, 64>(const LazyDecArgs&, hipStream_t);
template hipError_t lazy_decode_launch<F32, 128>(const LazyDecArgs&, hipStream_t);
}  // namespace fla
