// Lazy attention KV-cache (decode) forward instantiations for BF16 inputs.
#include "lazy_decode.inc"

namespace fla {
template hipError_t lazy_decode_launch<BF16, 32>(const LazyDecArgs&, hipStream_t);
template hipError_t lazy_decode_launch<BF16, 64>(const LazyDecArgs&, hipStream_t);
template hipError_t lazy_decode_launch<BF16, 128>(const LazyDecArgs&, hipStream_t);
}  // namespace fla
