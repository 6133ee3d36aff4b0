// Kernel argument blocks and launcher declarations shared by the C ABI (api.hip)
// and the per-dtype kernel translation units.
#pragma once
#include "common.h"

namespace fla {

struct AdaFwdArgs {
  Tensor4 q, k, v, o;
  float* tau;              // [B, H, L] threshold, (alpha-1)*score units
  float* wn;               // [B, H, L, D] sum U v / sum U, optional
  uint32_t* mask;          // [B, H, Tr, MW] block mask, optional
  const int32_t* varlen;   // [B], optional
  int B, H, L, Tr, MW;
  int G;                   // query heads per K/V head (K/V have H / G heads)
  float cz, beta;          // cz = (alpha-1)*scale, beta = 1/(alpha-1)
  int causal, skip, fb_maxit;
};

struct AdaBwdArgs {
  Tensor4 q, k, v, dout, dq, dk, dv;
  const float* tau;
  const float* wn;
  const uint32_t* mask;
  const int32_t* varlen;
  float* delta;            // [B, H, L] scratch
  int B, H, L, Tr, MW;
  int G;                   // query heads per K/V head
  float cz, beta, scale;
  int causal;
};

// Lazy bias entries staged in LDS per workgroup; distances >= LZ_SB read global memory.
static constexpr int LZ_SB = 1024;

struct LazyArgs {
  Tensor4 q, k, v, o, dout, dq, dk, dv;
  const float* bias;       // fp32 [H, bias_ld]
  int64_t bias_ld;
  const float* tau;        // fp32 [H]
  float* lse;              // [B, H, L]
  float* wdelta;           // [B, H, L, D], optional
  float* delta;            // [B, H, L] scratch (backward)
  const int32_t* varlen;
  float* dbias_part;       // [B*H*nQT, window] per-tile partials (backward, optional)
  float* dbias_far;        // [B*H*nQT*4, window - LZ_SB] per-wave partials of distances >= LZ_SB
  float* dtau_part;        // [B*H*nQT]
  float* dbias;            // [H, window]
  float* dtau;             // [H]
  uint32_t* mask;          // [B, H, ceil(L/64), MW] bits of (64-row, 64-key) blocks with e > 0, optional
  uint8_t* mask8;          // [B, H, ceil(L/64), ceil(L/64)] the same blocks, one byte each, optional
  int skip;                // skip the P V products of all-zero (wave, tile) pairs
  int MW;
  int B, H, L, W, nQT;
  int G;                   // query heads per K/V head
  int fold;                // workgroups per dispatch round (compute units); 0: plain order
  float scale;
};

// KV-cache (decode) forward of lazy attention.  A unit is (b, K/V head, group of RG query
// rows); row r of K/V head hk is query position r % Lq of query head hk*G + r / Lq.
struct LazyDecArgs {
  Tensor4 q, k, v, o;      // q, o [B, H, Lq, D]; k, v [B, H/G, Lk, D]
  const float* bias;       // fp32 [H, bias_ld]
  int64_t bias_ld;
  const float* tau;        // fp32 [H]
  const int32_t* varlen;   // [B] cache lengths, optional (else Lk)
  float* ml;               // [units, nsplit, RG, 2] per-chunk (max, sum exp2) scratch
  float* po;               // [units, nsplit, RG, D] per-chunk output scratch
  float* sc;               // optional [units, nsc, Lkp] base-2 score cache (matrix-core path)
  int B, H, G, Lq, Lk, W;
  int RG, nrg, nsplit, chunk;
  int nsc, Lkp;            // cached rows per unit, key stride of the cache (Lk rounded up to 32)
  float scale;
};

template <int DT, int D>
hipError_t ada_fwd_launch(const AdaFwdArgs& a, int mode, hipStream_t s);
template <int DT, int D>
hipError_t ada_bwd_launch(const AdaBwdArgs& a, int mode, hipStream_t s);
template <int DT, int D>
hipError_t lazy_fwd_launch(const LazyArgs& a, hipStream_t s);
template <int DT, int D>
hipError_t lazy_bwd_launch(const LazyArgs& a, hipStream_t s);

template <int DT, int D>
hipError_t lazy_decode_launch(const LazyDecArgs& a, hipStream_t s);

}  // namespace fla
