// Standalone row-wise alpha-entmax (forward and backward), one wave64 per row.
//
// Replaces the Triton kernel behind `triton_entmax(x, alpha, n_iter, fast_math)`
// (README.md:28-35; behaviour pinned by tests/test_triton_entmax.py).
//
// Threshold solver (shared with the attention kernels' row solver): in z = (alpha-1) x
// units, f(tau) = sum_j [z_j - tau]_+^beta - 1 with beta = 1/(alpha-1) is convex and
// decreasing, so Newton steps started below the root (tau0 = max z - 1, which always
// has f(tau0) >= 0) increase monotonically towards it and never overshoot.  For
// alpha = 2 and alpha = 1.5 the threshold on a fixed support has a closed form (linear /
// quadratic); once the closed-form root keeps every current support element positive it
// is the exact root and the iteration stops.  Other alphas stop when a Newton step no
// longer changes tau in fp32.  The output is renormalised to sum to one, like the
// entmax package's `ensure_sum_one`.
#include <type_traits>

#include "common.h"
#include "flashlazy_internal.h"

namespace fla {


// 16 bytes of a row <-> VEC = 16 / sizeof(T) floats.
template <int DT>
__device__ __forceinline__ void unpack16(const uint4& w, float* o) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  if constexpr (sizeof(typename Tr<DT>::T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __uint_as_float(u[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = Tr<DT>::to_f((typename Tr<DT>::T)(u[i] & 0xffffu));
      o[2 * i + 1] = Tr<DT>::to_f((typename Tr<DT>::T)(u[i] >> 16));
    }
  }
}
template <int DT>
__device__ __forceinline__ uint4 pack16(const float* v) {
  uint32_t u[4];
  if constexpr (sizeof(typename Tr<DT>::T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = __float_as_uint(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      u[i] = (uint32_t)Tr<DT>::from_f(v[2 * i]) | ((uint32_t)Tr<DT>::from_f(v[2 * i + 1]) << 16);
  }
  return make_uint4(u[0], u[1], u[2], u[3]);
}

// VIO: rows are read and written in 16-byte pieces (lane l holds elements
// (c*64 + l)*VEC .. +VEC-1 of chunk c); the launcher uses it when n, the row strides and the
// base pointers are multiples of 16 bytes.  The threshold only needs the row's values, not
// their order, so the solver is the same.
template <int DT, int EPL, int MODE, bool VIO = false>
__global__ __launch_bounds__(256) void entmax_fwd_kernel(const typename Tr<DT>::T* __restrict__ x,
                                                         typename Tr<DT>::T* __restrict__ y, int64_t rows, int n,
                                                         int64_t ldx, int64_t ldy, float alpha, float beta,
                                                         int maxit) {
  typedef typename Tr<DT>::T T;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * ldx;
  T* yr = y + row * ldy;
  const float am1 = alpha - 1.0f;
  constexpr int VEC = 16 / sizeof(T), NCH = EPL / VEC;
  float z[EPL];
  float m = -INFINITY;
  if constexpr (VIO) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int j0 = (c * 64 + lane) * VEC;
      if (j0 < n) {
        unpack16<DT>(*reinterpret_cast<const uint4*>(xr + j0), z + c * VEC);
#pragma unroll
        for (int v = 0; v < VEC; ++v) z[c * VEC + v] *= am1;
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) z[c * VEC + v] = -INFINITY;
      }
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) m = fmaxf(m, z[e]);
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      int j = e * 64 + lane;
      z[e] = j < n ? Tr<DT>::to_f(xr[j]) * am1 : -INFINITY;
      m = fmaxf(m, z[e]);
    }
  }
  m = wave_max(m);
  float tau = m - 1.0f;
  float F = 0.f, G = 0.f;
  for (int it = 0; it < maxit; ++it) {
    float K = 0.f, tmin = INFINITY;
    F = 0.f;
    G = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float t = z[e] - tau;
      if (t > 0.f) {
        float p, u;
        pow_pair<MODE>(t, beta, p, u);
        F += p;
        G += u;
        K += 1.f;
        tmin = fminf(tmin, t);
      }
    }
    F = wave_sum(F);
    G = wave_sum(G);
    K = wave_sum(K);
    tmin = wave_min(tmin);
    bool exact;
    float d = RowStep<MODE>::step(F, G, K, tmin, beta, exact);
    if (exact) {
      tau += d;
      break;
    }
    float nt = tau + d;
    if (!(nt > tau)) break;
    tau = nt;
  }
  // Final normaliser at the final tau.
  float S = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    float t = z[e] - tau, p = 0.f, u;
    if (t > 0.f) pow_pair<MODE>(t, beta, p, u);
    z[e] = p;
    S += p;
  }
  S = wave_sum(S);
  const float inv = 1.0f / S;
  if constexpr (VIO) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int j0 = (c * 64 + lane) * VEC;
      float o[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) o[v] = z[c * VEC + v] * inv;
      if (j0 < n) *reinterpret_cast<uint4*>(yr + j0) = pack16<DT>(o);
    }
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      int j = e * 64 + lane;
      if (j < n) yr[j] = Tr<DT>::from_f(z[e] * inv);
    }
  }
}

// Rows longer than 64*16 elements: the same solver, re-reading the row from global
// memory (L2-resident) on every pass.
template <int DT, int MODE>
__global__ __launch_bounds__(256) void entmax_fwd_stream_kernel(const typename Tr<DT>::T* __restrict__ x,
                                                                typename Tr<DT>::T* __restrict__ y, int64_t rows,
                                                                int n, int64_t ldx, int64_t ldy, float alpha,
                                                                float beta, int maxit) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const typename Tr<DT>::T* xr = x + row * ldx;
  typename Tr<DT>::T* yr = y + row * ldy;
  const float am1 = alpha - 1.0f;
  float m = -INFINITY;
  for (int j = lane; j < n; j += 64) m = fmaxf(m, Tr<DT>::to_f(xr[j]) * am1);
  m = wave_max(m);
  float tau = m - 1.0f;
  for (int it = 0; it < maxit; ++it) {
    float F = 0.f, G = 0.f, K = 0.f, tmin = INFINITY;
    for (int j = lane; j < n; j += 64) {
      float t = Tr<DT>::to_f(xr[j]) * am1 - tau;
      if (t > 0.f) {
        float p, u;
        pow_pair<MODE>(t, beta, p, u);
        F += p;
        G += u;
        K += 1.f;
        tmin = fminf(tmin, t);
      }
    }
    F = wave_sum(F);
    G = wave_sum(G);
    K = wave_sum(K);
    tmin = wave_min(tmin);
    bool exact;
    float d = RowStep<MODE>::step(F, G, K, tmin, beta, exact);
    if (exact) {
      tau += d;
      break;
    }
    float nt = tau + d;
    if (!(nt > tau)) break;
    tau = nt;
  }
  float S = 0.f;
  for (int j = lane; j < n; j += 64) {
    float t = Tr<DT>::to_f(xr[j]) * am1 - tau, p = 0.f, u;
    if (t > 0.f) pow_pair<MODE>(t, beta, p, u);
    S += p;
  }
  S = wave_sum(S);
  const float inv = 1.0f / S;
  for (int j = lane; j < n; j += 64) {
    float t = Tr<DT>::to_f(xr[j]) * am1 - tau, p = 0.f, u;
    if (t > 0.f) pow_pair<MODE>(t, beta, p, u);
    yr[j] = Tr<DT>::from_f(p * inv);
  }
}

// dx = U dy - (sum U dy / sum U) U,  U = y^(2-alpha) on y > 0 (entmax package backward).
template <int DT, int MODE>
__global__ __launch_bounds__(256) void entmax_bwd_kernel(const typename Tr<DT>::T* __restrict__ y,
                                                         const typename Tr<DT>::T* __restrict__ dy,
                                                         typename Tr<DT>::T* __restrict__ dx, int64_t rows, int n,
                                                         int64_t ldy, int64_t lddy, int64_t lddx, float alpha) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const typename Tr<DT>::T* yr = y + row * ldy;
  const typename Tr<DT>::T* gr = dy + row * lddy;
  typename Tr<DT>::T* xr = dx + row * lddx;
  auto U = [&](float yv) -> float {
    if (!(yv > 0.f)) return 0.f;
    if (MODE == 1) return sqrtf(yv);
    if (MODE == 2) return 1.f;
    return exp2f((2.0f - alpha) * log2f(yv));
  };
  float su = 0.f, sud = 0.f;
  for (int j = lane; j < n; j += 64) {
    float u = U(Tr<DT>::to_f(yr[j]));
    su += u;
    sud += u * Tr<DT>::to_f(gr[j]);
  }
  su = wave_sum(su);
  sud = wave_sum(sud);
  const float q = sud / su;
  for (int j = lane; j < n; j += 64) {
    float u = U(Tr<DT>::to_f(yr[j]));
    xr[j] = Tr<DT>::from_f(u * (Tr<DT>::to_f(gr[j]) - q));
  }
}

template <int DT, int MODE>
static hipError_t launch_fwd(const void* x, void* y, int64_t rows, int n, int64_t ldx, int64_t ldy, float alpha,
                             int maxit, hipStream_t s) {
  typedef typename Tr<DT>::T T;
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  const float beta = 1.0f / (alpha - 1.0f);
  const T* xp = (const T*)x;
  T* yp = (T*)y;
  constexpr int VEC = 16 / sizeof(T);
  const bool vio = n % VEC == 0 && ldx % VEC == 0 && ldy % VEC == 0 && (uintptr_t)x % 16 == 0 &&
                   (uintptr_t)y % 16 == 0;
  auto go = [&](auto epl_tag) {
    constexpr int EPL = decltype(epl_tag)::value;
    if constexpr (EPL % VEC == 0) {
      if (vio) {
        hipLaunchKernelGGL((entmax_fwd_kernel<DT, EPL, MODE, true>), grid, block, 0, s, xp, yp, rows, n, ldx, ldy,
                           alpha, beta, maxit);
        return;
      }
    }
    hipLaunchKernelGGL((entmax_fwd_kernel<DT, EPL, MODE, false>), grid, block, 0, s, xp, yp, rows, n, ldx, ldy,
                       alpha, beta, maxit);
  };
  if (n <= 64)
    go(std::integral_constant<int, 1>{});
  else if (n <= 128)
    go(std::integral_constant<int, 2>{});
  else if (n <= 256)
    go(std::integral_constant<int, 4>{});
  else if (n <= 512)
    go(std::integral_constant<int, 8>{});
  else if (n <= 1024)
    go(std::integral_constant<int, 16>{});
  else
    hipLaunchKernelGGL((entmax_fwd_stream_kernel<DT, MODE>), grid, block, 0, s, xp, yp, rows, n, ldx, ldy, alpha, beta, maxit);
  return hipGetLastError();
}

template <int DT>
static hipError_t dispatch_fwd(const void* x, void* y, int64_t rows, int n, int64_t ldx, int64_t ldy, float alpha,
                               int maxit, hipStream_t s) {
  int mode = alpha_mode(alpha);
  if (mode == 1) return launch_fwd<DT, 1>(x, y, rows, n, ldx, ldy, alpha, maxit, s);
  if (mode == 2) return launch_fwd<DT, 2>(x, y, rows, n, ldx, ldy, alpha, maxit, s);
  return launch_fwd<DT, 0>(x, y, rows, n, ldx, ldy, alpha, maxit, s);
}

template <int DT>
static hipError_t dispatch_bwd(const void* y, const void* dy, void* dx, int64_t rows, int n, int64_t ldy,
                               int64_t lddy, int64_t lddx, float alpha, hipStream_t s) {
  typedef typename Tr<DT>::T T;
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  int mode = alpha_mode(alpha);
  const T* yp = (const T*)y;
  const T* gp = (const T*)dy;
  T* xp = (T*)dx;
  if (mode == 1)
    hipLaunchKernelGGL((entmax_bwd_kernel<DT, 1>), grid, block, 0, s, yp, gp, xp, rows, n, ldy, lddy, lddx, alpha);
  else if (mode == 2)
    hipLaunchKernelGGL((entmax_bwd_kernel<DT, 2>), grid, block, 0, s, yp, gp, xp, rows, n, ldy, lddy, lddx, alpha);
  else
    hipLaunchKernelGGL((entmax_bwd_kernel<DT, 0>), grid, block, 0, s, yp, gp, xp, rows, n, ldy, lddy, lddx, alpha);
  return hipGetLastError();
}

}  // namespace fla

using namespace fla;

extern "C" int fla_entmax_fwd(const void* x, void* y, int64_t rows, int64_t n, int64_t ldx, int64_t ldy, int dtype,
                              float alpha, int n_iter, int fast_math, void* stream_) {
  (void)fast_math;
  hipStream_t stream = (hipStream_t)stream_;
  if (rows < 0 || n <= 0 || n > (int64_t)1 << 30 || !(alpha > 1.0f) || alpha > 2.0f || !x || !y) return FLA_EINVAL;
  if (rows == 0) return 0;
  // The solver runs to fp32 convergence; n_iter only raises the iteration cap.
  int maxit = n_iter > 100 ? n_iter : 100;
  hipError_t e;
  switch (dtype) {
    case F32: e = dispatch_fwd<F32>(x, y, rows, (int)n, ldx, ldy, alpha, maxit, stream); break;
    case F16: e = dispatch_fwd<F16>(x, y, rows, (int)n, ldx, ldy, alpha, maxit, stream); break;
    case BF16: e = dispatch_fwd<BF16>(x, y, rows, (int)n, ldx, ldy, alpha, maxit, stream); break;
    default: return FLA_EINVAL;
  }
  return (int)e;
}

extern "C" int fla_entmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t n, int64_t ldy,
                              int64_t lddy, int64_t lddx, int dtype, float alpha, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (rows < 0 || n <= 0 || n > (int64_t)1 << 30 || !(alpha > 1.0f) || alpha > 2.0f || !y || !dy || !dx) return FLA_EINVAL;
  if (rows == 0) return 0;
  hipError_t e;
  switch (dtype) {
    case F32: e = dispatch_bwd<F32>(y, dy, dx, rows, (int)n, ldy, lddy, lddx, alpha, stream); break;
    case F16: e = dispatch_bwd<F16>(y, dy, dx, rows, (int)n, ldy, lddy, lddx, alpha, stream); break;
    case BF16: e = dispatch_bwd<BF16>(y, dy, dx, rows, (int)n, ldy, lddy, lddx, alpha, stream); break;
    default: return FLA_EINVAL;
  }
  return (int)e;
}
