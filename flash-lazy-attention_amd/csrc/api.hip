// C ABI entry points (declared in include/flashlazy.h): argument validation and dispatch
// on dtype / head dim / alpha.  Nothing here allocates; all launches are asynchronous on
// the caller's stream.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "args.h"
#include "flashlazy_internal.h"

#ifndef FLA_FOLD_VALUE
#define FLA_FOLD_VALUE cu_count()
#endif

using namespace fla;

namespace {

int elem_size(int dtype) { return dtype == FLA_F32 ? 4 : 2; }

bool good_tensor(const fla_tensor4_t* t, int dtype) {
  if (!t || !t->data) return false;
  const int es = elem_size(dtype);
  if (((uintptr_t)t->data) % 16) return false;
  if ((t->stride_b * es) % 16 || (t->stride_h * es) % 16 || (t->stride_l * es) % 16) return false;
  // tiles are read with 32-bit buffer offsets: 64 rows of stride_l must stay far below 2 GiB
  if (t->stride_l <= 0 || t->stride_l * es > (1 << 24)) return false;
  return true;
}

Tensor4 T4(const fla_tensor4_t* t) {
  Tensor4 r;
  r.data = t->data;
  r.sb = t->stride_b;
  r.sh = t->stride_h;
  r.sl = t->stride_l;
  return r;
}

bool good_common(int B, int H, int L, int D, int dtype) {
  if (B <= 0 || H <= 0 || L <= 0 || L > (1 << 17)) return false;
  if (D != 32 && D != 64 && D != 128) return false;
  if (dtype != FLA_F32 && dtype != FLA_F16 && dtype != FLA_BF16) return false;
  if ((int64_t)B * H * ((L + 127) / 128) > 0x7fffffffLL) return false;
  return true;
}


}  // namespace

#define FLA_DISPATCH(LAUNCH, ARGS, ...)                                           \
  switch (dtype * 1000 + D) {                                                     \
    case FLA_F32 * 1000 + 32: e = LAUNCH<F32, 32>(ARGS, ##__VA_ARGS__); break;    \
    case FLA_F32 * 1000 + 64: e = LAUNCH<F32, 64>(ARGS, ##__VA_ARGS__); break;    \
    case FLA_F32 * 1000 + 128: e = LAUNCH<F32, 128>(ARGS, ##__VA_ARGS__); break;  \
    case FLA_F16 * 1000 + 32: e = LAUNCH<F16, 32>(ARGS, ##__VA_ARGS__); break;    \
    case FLA_F16 * 1000 + 64: e = LAUNCH<F16, 64>(ARGS, ##__VA_ARGS__); break;    \
    case FLA_F16 * 1000 + 128: e = LAUNCH<F16, 128>(ARGS, ##__VA_ARGS__); break;  \
    case FLA_BF16 * 1000 + 32: e = LAUNCH<BF16, 32>(ARGS, ##__VA_ARGS__); break;  \
    case FLA_BF16 * 1000 + 64: e = LAUNCH<BF16, 64>(ARGS, ##__VA_ARGS__); break;  \
    case FLA_BF16 * 1000 + 128: e = LAUNCH<BF16, 128>(ARGS, ##__VA_ARGS__); break; \
    default: return FLA_EUNSUPPORTED;                                             \
  }

namespace {
// Compute units of the current device (cached per device; 0 if the query fails).  Concurrent
// first calls may both query; they store the same value.
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}
}  // namespace

extern "C" const char* fla_version(void) { return "flashlazy-gfx950 0.1.0"; }

extern "C" int fla_adasplash_mask_words(int L) {
  if (L <= 0) return 0;
  const int tc = (L + 63) / 64;
  return (tc + 31) / 32;
}

namespace {
__global__ void __launch_bounds__(256) unpack_mask_kernel(const uint32_t* __restrict__ words, uint8_t* __restrict__ out,
                                                          int64_t n, int mw, int ncols) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = i / ncols;
  const int c = (int)(i - r * ncols);
  out[i] = (uint8_t)((words[r * mw + (c >> 5)] >> (c & 31)) & 1u);
}
}  // namespace

extern "C" int fla_unpack_block_mask(const uint32_t* words, uint8_t* out, int64_t rows, int mw, int ncols,
                                     void* stream) {
  if (rows < 0 || mw <= 0 || ncols < 0 || ncols > 32 * mw) return FLA_EINVAL;
  const int64_t n = rows * ncols;
  if (n == 0) return FLA_OK;
  if (!words || !out) return FLA_EINVAL;
  const int64_t nb = (n + 255) / 256;
  if (nb > 0x7fffffffLL) return FLA_EINVAL;
  hipLaunchKernelGGL(unpack_mask_kernel, dim3((unsigned)nb), dim3(256), 0, (hipStream_t)stream, words, out, n, mw,
                     ncols);
  return (int)hipGetLastError();
}

extern "C" int fla_adasplash_fwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                                 const fla_tensor4_t* out, float* tau, float* wn, uint32_t* block_mask,
                                 const int32_t* varlen, int B, int H, int Hkv, int L, int D, int dtype, float alpha, int niter,
                                 int is_causal, int skip_empty_blocks, float scale, void* stream) {
  if (!good_common(B, H, L, D, dtype)) return FLA_EINVAL;
  if (Hkv <= 0 || H % Hkv) return FLA_EINVAL;
  if (!good_tensor(q, dtype) || !good_tensor(k, dtype) || !good_tensor(v, dtype) || !good_tensor(out, dtype))
    return FLA_EINVAL;
  if (!tau || !(alpha > 1.0f) || alpha > 2.0f || !(scale > 0.0f)) return FLA_EINVAL;
  AdaFwdArgs a;
  a.q = T4(q);
  a.k = T4(k);
  a.v = T4(v);
  a.o = T4(out);
  a.tau = tau;
  a.wn = wn;
  a.mask = block_mask;
  a.varlen = varlen;
  a.B = B;
  a.H = H;
  a.G = H / Hkv;
  a.L = L;
  a.Tr = (L + 127) / 128;
  a.MW = fla_adasplash_mask_words(L);
  a.cz = (alpha - 1.0f) * scale;
  a.beta = 1.0f / (alpha - 1.0f);
  a.causal = is_causal ? 1 : 0;
  a.skip = skip_empty_blocks ? 1 : 0;
  a.fb_maxit = niter > 100 ? niter : 100;
  const int mode = alpha_mode(alpha);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  FLA_DISPATCH(ada_fwd_launch, a, mode, s)
  return (int)e;
}

extern "C" int fla_adasplash_bwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                                 const fla_tensor4_t* dout, const fla_tensor4_t* dq, const fla_tensor4_t* dk,
                                 const fla_tensor4_t* dv, const float* tau, const float* wn,
                                 const uint32_t* block_mask, const int32_t* varlen, float* delta_ws, int B, int H, int Hkv,
                                 int L, int D, int dtype, float alpha, int is_causal, float scale, void* stream) {
  if (!good_common(B, H, L, D, dtype)) return FLA_EINVAL;
  if (Hkv <= 0 || H % Hkv) return FLA_EINVAL;
  if (!good_tensor(q, dtype) || !good_tensor(k, dtype) || !good_tensor(v, dtype) || !good_tensor(dout, dtype) ||
      !good_tensor(dq, dtype) || !good_tensor(dk, dtype) || !good_tensor(dv, dtype))
    return FLA_EINVAL;
  if (!tau || !wn || !delta_ws || !(alpha > 1.0f) || alpha > 2.0f || !(scale > 0.0f)) return FLA_EINVAL;
  AdaBwdArgs a;
  a.q = T4(q);
  a.k = T4(k);
  a.v = T4(v);
  a.dout = T4(dout);
  a.dq = T4(dq);
  a.dk = T4(dk);
  a.dv = T4(dv);
  a.tau = tau;
  a.wn = wn;
  a.mask = block_mask;
  a.varlen = varlen;
  a.delta = delta_ws;
  a.B = B;
  a.H = H;
  a.G = H / Hkv;
  a.L = L;
  a.Tr = (L + 127) / 128;
  a.MW = fla_adasplash_mask_words(L);
  a.cz = (alpha - 1.0f) * scale;
  a.beta = 1.0f / (alpha - 1.0f);
  a.scale = scale;
  a.causal = is_causal ? 1 : 0;
  const int mode = alpha_mode(alpha);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  FLA_DISPATCH(ada_bwd_launch, a, mode, s)
  return (int)e;
}

extern "C" size_t fla_lazy_bwd_workspace_size(int B, int H, int L, int window) {
  if (B <= 0 || H <= 0 || L <= 0 || window <= 0) return 0;
  const size_t nqt = (size_t)(L + 127) / 128;
  const size_t parts = (size_t)B * H * nqt;
  // dbias partials, dtau partials, delta [B, H, L], per-wave dbias partials of distances
  // >= LZ_SB; each region 256-byte aligned.
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const size_t nfar = window > LZ_SB ? (size_t)(window - LZ_SB) : 0;
  return up(parts * (size_t)window * 4) + up(parts * 4) + up((size_t)B * H * L * 4) + up(parts * 4 * nfar * 4);
}

extern "C" int fla_lazy_fwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                            const fla_tensor4_t* out, const float* bias, int64_t bias_ld, const float* tau,
                            int window, float* lse, float* wdelta, uint32_t* block_mask, uint8_t* block_mask_u8,
                            int skip_empty_blocks,
                            const int32_t* varlen, int B, int H, int Hkv, int L, int D,
                            int dtype, float scale, void* stream) {
  if (!good_common(B, H, L, D, dtype)) return FLA_EINVAL;
  if (Hkv <= 0 || H % Hkv) return FLA_EINVAL;
  if (!good_tensor(q, dtype) || !good_tensor(k, dtype) || !good_tensor(v, dtype) || !good_tensor(out, dtype))
    return FLA_EINVAL;
  if (!bias || !tau || !lse || window <= 0 || bias_ld < window || !(scale > 0.0f)) return FLA_EINVAL;
  LazyArgs a = {};
  a.q = T4(q);
  a.k = T4(k);
  a.v = T4(v);
  a.o = T4(out);
  a.bias = bias;
  a.bias_ld = bias_ld;
  a.tau = tau;
  a.lse = lse;
  a.wdelta = wdelta;
  a.mask = block_mask;
  a.mask8 = block_mask_u8;
  a.skip = skip_empty_blocks ? 1 : 0;
  a.MW = fla_adasplash_mask_words(L);
  a.varlen = varlen;
  a.B = B;
  a.H = H;
  a.G = H / Hkv;
  a.L = L;
  a.W = window;
  a.nQT = (L + 127) / 128;
  a.fold = FLA_FOLD_VALUE;
  a.scale = scale;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  FLA_DISPATCH(lazy_fwd_launch, a, s)
  return (int)e;
}

extern "C" int fla_lazy_bwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                            const fla_tensor4_t* dout, const fla_tensor4_t* dq, const fla_tensor4_t* dk,
                            const fla_tensor4_t* dv, const float* bias, int64_t bias_ld, const float* tau, int window,
                            const float* lse, const float* wdelta, const int32_t* varlen, float* dbias, float* dtau,
                            void* workspace, size_t workspace_bytes, int B, int H, int Hkv, int L, int D, int dtype,
                            float scale, void* stream) {
  if (!good_common(B, H, L, D, dtype)) return FLA_EINVAL;
  if (Hkv <= 0 || H % Hkv) return FLA_EINVAL;
  if (!good_tensor(q, dtype) || !good_tensor(k, dtype) || !good_tensor(v, dtype) || !good_tensor(dout, dtype) ||
      !good_tensor(dq, dtype) || !good_tensor(dk, dtype) || !good_tensor(dv, dtype))
    return FLA_EINVAL;
  if (!bias || !tau || !lse || !wdelta || window <= 0 || bias_ld < window || !(scale > 0.0f)) return FLA_EINVAL;
  if ((dbias == nullptr) != (dtau == nullptr)) return FLA_EINVAL;
  const size_t need = fla_lazy_bwd_workspace_size(B, H, L, window);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace) % 256) return FLA_EWORKSPACE;
  LazyArgs a = {};
  a.q = T4(q);
  a.k = T4(k);
  a.v = T4(v);
  a.dout = T4(dout);
  a.dq = T4(dq);
  a.dk = T4(dk);
  a.dv = T4(dv);
  a.bias = bias;
  a.bias_ld = bias_ld;
  a.tau = tau;
  a.lse = const_cast<float*>(lse);
  a.wdelta = const_cast<float*>(wdelta);
  a.varlen = varlen;
  a.B = B;
  a.H = H;
  a.G = H / Hkv;
  a.L = L;
  a.W = window;
  a.nQT = (L + 127) / 128;
  a.fold = FLA_FOLD_VALUE;
  a.scale = scale;
  const size_t parts = (size_t)B * H * a.nQT;
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  char* ws = (char*)workspace;
  a.dbias_part = (float*)ws;
  a.dtau_part = (float*)(ws + up(parts * (size_t)window * 4));
  a.delta = (float*)(ws + up(parts * (size_t)window * 4) + up(parts * 4));
  a.dbias_far = (float*)(ws + up(parts * (size_t)window * 4) + up(parts * 4) + up((size_t)B * H * L * 4));
  a.dbias = dbias;
  a.dtau = dtau;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  FLA_DISPATCH(lazy_bwd_launch, a, s)
  return (int)e;
}

namespace {

// Decode work split: query rows in groups of RG, keys in chunks of a multiple of 64 chosen so
// that units x chunks gives about 512 (matrix-core) or 1024 (vector kernels) workgroups.
// 16-bit inputs use the matrix-core kernels (RG = 32); fp32 inputs the vector kernels with
// RG = 1, 2, 4 or 8.
struct DecPlan {
  int G, RG, nrg, nsplit, chunk, nsc, Lkp;
  size_t ml_bytes, po_bytes, sc_bytes;
  size_t bytes() const { return ml_bytes + po_bytes + sc_bytes; }
};

bool dec_plan(int B, int H, int Hkv, int Lq, int Lk, int D, bool mfma, DecPlan& p) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || Lq <= 0 || Lk <= 0 || Lk > (1 << 24)) return false;
  if (D != 32 && D != 64 && D != 128) return false;
  p.G = H / Hkv;
  const int64_t R = (int64_t)p.G * Lq;
  if (R > (1 << 20)) return false;
  p.RG = mfma ? 32 : R >= 8 ? 8 : R >= 4 ? 4 : R >= 2 ? 2 : 1;
  p.nrg = (int)((R + p.RG - 1) / p.RG);
  const int64_t units = (int64_t)B * Hkv * p.nrg;
  const int64_t maxsplit = (Lk + 255) / 256;
  // workgroups to aim for: the matrix-core kernels run two per compute unit, and one full round
  // on MI355X's 256 units measured 5-11% faster than two (1024); the vector kernels keep 1024
  const int64_t target = mfma ? 512 : 1024;
  int64_t ns = (target + units - 1) / units;
  ns = ns < 1 ? 1 : (ns > maxsplit ? maxsplit : ns);
  p.chunk = (int)(((Lk + ns - 1) / ns + 63) / 64 * 64);
  p.nsplit = (Lk + p.chunk - 1) / p.chunk;
  if (units * p.nsplit > 0x7fffffffLL) return false;
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  p.ml_bytes = up((size_t)units * p.nsplit * p.RG * 2 * 4);
  p.po_bytes = up((size_t)units * p.nsplit * p.RG * D * 4);
  // Score cache of the matrix-core path: 4 bytes per key and row written and read back instead
  // of reading a 2*D-byte key row again; kept when that halves the re-read at least (fewer
  // than D/4 rows per unit, so at most half the size of K).
  p.nsc = 0;
  p.Lkp = (Lk + 31) / 32 * 32;
  if (p.RG == 32) {
    const int rows = (int)(R < 32 ? R : 32);
    if (4 * rows < D) p.nsc = rows;
  }
  p.sc_bytes = up((size_t)units * p.nsc * p.Lkp * 4);
  return true;
}

}  // namespace

extern "C" size_t fla_lazy_decode_workspace_size(int B, int H, int Hkv, int Lq, int Lk, int D) {
  // the larger of the two kernel families' needs, so that the size does not depend on dtype
  DecPlan p, pm;
  if (!dec_plan(B, H, Hkv, Lq, Lk, D, false, p) || !dec_plan(B, H, Hkv, Lq, Lk, D, true, pm)) return 0;
  return std::max(p.bytes(), pm.bytes());
}

// Static scratch of fla_lazy_decode_fwd_static: one copy per GPU, held until the process ends.
// Host code never uses the name `scratch` as an address (on the host it is only a stand-in
// for the device symbol): the device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) char scratch[FLA_STATIC_SCRATCH_BYTES];

namespace {

int lazy_decode(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v, const fla_tensor4_t* out,
                const float* bias, int64_t bias_ld, const float* tau, int window, const int32_t* varlen,
                void* workspace, size_t workspace_bytes, int B, int H, int Hkv, int Lq, int Lk, int D, int dtype,
                float scale, void* stream) {
  if (dtype != FLA_F32 && dtype != FLA_F16 && dtype != FLA_BF16) return FLA_EUNSUPPORTED;
  DecPlan p;
  if (!dec_plan(B, H, Hkv, Lq, Lk, D, dtype != FLA_F32, p)) return FLA_EINVAL;
  if (!good_tensor(q, dtype) || !good_tensor(k, dtype) || !good_tensor(v, dtype) || !good_tensor(out, dtype))
    return FLA_EINVAL;
  if (!bias || !tau || window <= 0 || bias_ld < window || !(scale > 0.0f)) return FLA_EINVAL;
  if (!workspace || workspace_bytes < p.bytes() || ((uintptr_t)workspace) % 256) return FLA_EWORKSPACE;
  LazyDecArgs a = {};
  a.q = T4(q);
  a.k = T4(k);
  a.v = T4(v);
  a.o = T4(out);
  a.bias = bias;
  a.bias_ld = bias_ld;
  a.tau = tau;
  a.varlen = varlen;
  a.ml = (float*)workspace;
  a.po = (float*)((char*)workspace + p.ml_bytes);
  a.sc = p.nsc ? (float*)((char*)workspace + p.ml_bytes + p.po_bytes) : nullptr;
  a.nsc = p.nsc;
  a.Lkp = p.Lkp;
  a.B = B;
  a.H = H;
  a.G = p.G;
  a.Lq = Lq;
  a.Lk = Lk;
  a.W = window;
  a.RG = p.RG;
  a.nrg = p.nrg;
  a.nsplit = p.nsplit;
  a.chunk = p.chunk;
  a.scale = scale;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  FLA_DISPATCH(lazy_decode_launch, a, s)
  return (int)e;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // guarded by g_scratch_mu

// Device address of the current device's scratch (resolved on the first call per device).
int static_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return FLA_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int fla_lazy_decode_fwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                                   const fla_tensor4_t* out, const float* bias, int64_t bias_ld, const float* tau,
                                   int window, const int32_t* varlen, void* workspace, size_t workspace_bytes, int B,
                                   int H, int Hkv, int Lq, int Lk, int D, int dtype, float scale, void* stream) {
  return lazy_decode(q, k, v, out, bias, bias_ld, tau, window, varlen, workspace, workspace_bytes, B, H, Hkv, Lq, Lk,
                     D, dtype, scale, stream);
}

extern "C" int fla_lazy_decode_fwd_static(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                                          const fla_tensor4_t* out, const float* bias, int64_t bias_ld,
                                          const float* tau, int window, const int32_t* varlen, int B, int H, int Hkv,
                                          int Lq, int Lk, int D, int dtype, float scale, void* stream) {
  const size_t need = fla_lazy_decode_workspace_size(B, H, Hkv, Lq, Lk, D);
  if (need == 0) return FLA_EINVAL;
  if (need > FLA_STATIC_SCRATCH_BYTES) return FLA_EWORKSPACE;
  void* ws = nullptr;
  const int rc = static_scratch(&ws);
  if (rc != 0) return rc;
  // Every scratch byte the kernels read is written earlier in the same call: nothing to clear.
  return lazy_decode(q, k, v, out, bias, bias_ld, tau, window, varlen, ws, FLA_STATIC_SCRATCH_BYTES, B, H, Hkv, Lq,
                     Lk, D, dtype, scale, stream);
}
