// Shared device helpers for the gfx950 (MI355X, CDNA4) kernels of this library.
//
// Conventions used by every attention kernel:
//  * wave64; a 256-thread workgroup is 4 waves.
//  * Matrix products use the 32x32 MFMA family.  For C[32][32] += A[32][K] B[K][32]
//    lane l supplies row (l%32) of A and column (l%32) of B, each as KPL consecutive
//    "k slots", and lane group g = l/32 selects which slots.  The accumulator holds
//    column (l%32) and the 16 rows  row_of(r, g) = 8*(r/4) + 4*g + (r%4),  r = 0..15.
//  * When an accumulator is fed back as the B operand of the next product (P^T, dS^T ...)
//    the contraction index of register r is row_of(r, g).  The A operand of that product
//    is then read with the same mapping, so the pairing of k slots between A and B is a
//    permutation shared by both operands and the sum over k is unchanged.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fla {

enum DType : int { F32 = 0, F16 = 1, BF16 = 2 };

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ constexpr int row_of(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// Element type traits: storage type, MFMA fragment type, k slots per lane.
template <int DT>
struct Tr;

template <>
struct Tr<BF16> {
  typedef uint16_t T;
  typedef bf16x8 frag;
  static constexpr int KPL = 8;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f(T x) { return __uint_as_float(((uint32_t)x) << 16); }
  static __device__ __forceinline__ T from_f(float x) {
    __bf16 h = (__bf16)x;
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ void set(frag& f, int e, float x) { f[e] = (__bf16)x; }
  static __device__ __forceinline__ void set_raw(frag& f, int e, T x) { f[e] = __builtin_bit_cast(__bf16, x); }
  static __device__ __forceinline__ frag zero() { frag f; for (int e = 0; e < 8; ++e) f[e] = (__bf16)0.0f; return f; }
};

template <>
struct Tr<F16> {
  typedef uint16_t T;
  typedef f16x8 frag;
  static constexpr int KPL = 8;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f(T x) { return (float)__builtin_bit_cast(_Float16, x); }
  static __device__ __forceinline__ T from_f(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
  static __device__ __forceinline__ void set(frag& f, int e, float x) { f[e] = (_Float16)x; }
  static __device__ __forceinline__ void set_raw(frag& f, int e, T x) { f[e] = __builtin_bit_cast(_Float16, x); }
  static __device__ __forceinline__ frag zero() { frag f; for (int e = 0; e < 8; ++e) f[e] = (_Float16)0.0f; return f; }
};

template <>
struct Tr<F32> {
  typedef float T;
  typedef float frag;
  static constexpr int KPL = 1;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f(T x) { return x; }
  static __device__ __forceinline__ T from_f(float x) { return x; }
  static __device__ __forceinline__ void set(frag& f, int, float x) { f = x; }
  static __device__ __forceinline__ void set_raw(frag& f, int, T x) { f = x; }
  static __device__ __forceinline__ frag zero() { return 0.0f; }
};

// Load KPL consecutive elements (16 bytes for 16-bit types) as one fragment.
template <int DT>
__device__ __forceinline__ typename Tr<DT>::frag load_frag(const typename Tr<DT>::T* p) {
  return *reinterpret_cast<const typename Tr<DT>::frag*>(p);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Cross-lane helpers (wave64).
__device__ __forceinline__ float pair_sum(float x) { return x + __shfl_xor(x, 32); }
__device__ __forceinline__ float pair_max(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
__device__ __forceinline__ float pair_min(float x) { return fminf(x, __shfl_xor(x, 32)); }

// Whole-wave reductions, every lane gets the result.  Within a row of 16 lanes the four
// exchange steps are DPP operand modifiers of the VALU op itself (quad permutations for lane
// xor 1 and 2; once the 4 lanes of a quad agree, the half-row mirror pairs quad q with quad
// q ^ 1 and the row mirror pairs the two halves of the row); the xor-16 and xor-32 steps cross
// rows through the LDS crossbar.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <typename Op>
__device__ __forceinline__ float wave_reduce(float x, Op op) {
  x = op(x, dpp_f<0xB1>(x));   // quad_perm [1,0,3,2]: lane ^ 1
  x = op(x, dpp_f<0x4E>(x));   // quad_perm [2,3,0,1]: lane ^ 2
  x = op(x, dpp_f<0x141>(x));  // row_half_mirror: quad pairs within 8 lanes
  x = op(x, dpp_f<0x140>(x));  // row_mirror: the two 8-lane halves of a row
  x = op(x, __shfl_xor(x, 16));
  x = op(x, __shfl_xor(x, 32));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
  return wave_reduce(x, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float x) {
  return wave_reduce(x, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_min(float x) {
  return wave_reduce(x, [](float a, float b) { return fminf(a, b); });
}

// t^beta and t^(beta-1) for t > 0.  MODE 1: alpha = 1.5 (beta = 2), MODE 2: alpha = 2
// (beta = 1), MODE 0: any alpha in (1, 2] via exp2/log2.
template <int MODE>
__device__ __forceinline__ void pow_pair(float t, float beta, float& p, float& u) {
  if (MODE == 1) {
    p = t * t;
    u = t;
  } else if (MODE == 2) {
    p = t;
    u = 1.0f;
  } else {
    float lg = __builtin_amdgcn_logf(t);  // log2
    u = __builtin_amdgcn_exp2f((beta - 1.0f) * lg);
    p = u * t;
  }
}

// Threshold solver step shared by every entmax kernel.  In z = (alpha-1)*score units
// f(tau) = sum_j [z_j - tau]_+^beta - 1 is convex and decreasing, so Newton steps from
// below the root never overshoot; for alpha = 1.5 / 2 the closed-form root on the current
// support is exact once it keeps every support element positive.
template <int MODE>
struct RowStep {
  // One solver step from sums over t = z - tau > 0: F = sum t^beta, G = sum t^(beta-1),
  // K = count, tmin = smallest positive t.  Returns the step; sets `exact` when
  // tau + step is the exact root (MODE 1/2).
  static __device__ __forceinline__ float step(float F, float G, float K, float tmin, float beta, bool& exact) {
    exact = false;
    if (MODE == 1) {
      // sum_S (t - d)^2 = 1  ->  K d^2 - 2 G d + F - 1 = 0, smaller root.
      float disc = fmaxf(G * G - K * (F - 1.0f), 0.0f);
      float d = (F - 1.0f) / (G + sqrtf(disc));
      if (d < tmin) { exact = true; return d; }
      return (F - 1.0f) / (2.0f * G);
    } else if (MODE == 2) {
      float d = (F - 1.0f) / K;
      if (d < tmin) exact = true;
      return d;
    } else {
      return (F - 1.0f) / (beta * G);
    }
  }
};

// Stage a [ROWS][D] tile of T (global row stride `ld`, rows >= nvalid zero-filled)
// into LDS with row stride LDR elements.  16-byte vector moves, all 256 threads.
template <typename T, int ROWS, int D, int LDR>
__device__ __forceinline__ void stage_rows(T* __restrict__ lds, const T* __restrict__ g, int64_t ld, int nvalid, int tid) {
  constexpr int EPV = 16 / sizeof(T);
  constexpr int CPR = D / EPV;
  constexpr int NCH = ROWS * CPR;
#pragma unroll
  for (int c = tid; c < NCH; c += 256) {
    int row = c / CPR, col = (c % CPR) * EPV;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < nvalid) v = *reinterpret_cast<const uint4*>(g + row * ld + col);
    *reinterpret_cast<uint4*>(lds + row * LDR + col) = v;
  }
}

// Stage a [ROWS][D] global tile transposed into LDS as [D][ROWS] with row stride LDR.
template <typename T, int ROWS, int D, int LDR>
__device__ __forceinline__ void stage_rows_t(T* __restrict__ lds, const T* __restrict__ g, int64_t ld, int nvalid, int tid) {
  constexpr int EPV = 16 / sizeof(T);
  constexpr int CPR = D / EPV;
  constexpr int NCH = ROWS * CPR;
#pragma unroll
  for (int c = tid; c < NCH; c += 256) {
    int row = c % ROWS, col = (c / ROWS) * EPV;
    union { uint4 v; T e[EPV]; } u;
    u.v = make_uint4(0, 0, 0, 0);
    if (row < nvalid) u.v = *reinterpret_cast<const uint4*>(g + row * ld + col);
#pragma unroll
    for (int e = 0; e < EPV; ++e) lds[(col + e) * LDR + row] = u.e[e];
  }
}

// max(x, 0) as an integer max on the bit pattern (every negative float, -0 and -inf included,
// has a negative pattern).  One v_max_i32, where fmaxf on an MFMA result would first
// canonicalise its operand.  x must not be NaN.
__device__ __forceinline__ float pos_part(float x) { return __int_as_float(max(__float_as_int(x), 0)); }
// Whether any of the 32 values is > 0 (same bit-pattern argument: positive floats are exactly
// the positive patterns).
__device__ __forceinline__ bool any_pos(const f32x16& a, const f32x16& b) {
  int m = 0;
#pragma unroll
  for (int r = 0; r < 16; ++r) m = max(m, max(__float_as_int(a[r]), __float_as_int(b[r])));
  return m > 0;
}

// t = (alpha-1)*scale*s - tau as one fused multiply-add (threshold search over stored scores).
// The sweeps that produce p for the output and the gradients (forward pass B, both backward
// kernels) instead start the q.k MFMA from -tau/cz, all with the same fp32 value, so they agree
// with each other on the support and the block mask.
__device__ __forceinline__ float zt(float s, float cz, float tau) { return __builtin_fmaf(s, cz, -tau); }

// Buffer resource over [base, base + bytes): raw buffer loads past the end return zero, which
// zero-fills tile rows beyond the valid sequence length without any per-lane test.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
// s_waitcnt vmcnt(0): wait for every outstanding vector-memory load of this wave.
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Bytes covering rows [0, nvalid) of a tile with row stride ld and D columns.
template <typename T, int D>
__device__ __forceinline__ uint32_t tile_bytes(int64_t ld, int nvalid) {
  return nvalid > 0 ? (uint32_t)(((int64_t)(nvalid - 1) * ld + D) * sizeof(T)) : 0u;
}

// Row-major LDS layout for 16-bit tiles that are read both by rows (16-byte reads, 16 lanes per
// LDS cycle) and with the transposing read (8 bytes per lane, 32 lanes per cycle).  Row r starts
// at element r * D + 8 * shift(r): rows are packed and shifted by whole 16-byte slots so that,
// with 64 four-byte banks (16 slots of 16 bytes), (a) one 16-byte column of 16 consecutive rows
// (from a multiple of 16) covers all 16 slots and (b) 64 bytes of columns (from a multiple of 64
// bytes) of 4 consecutive rows (from a multiple of 4) cover all 16 slots.  A constant row stride
// cannot do both for D = 32, 64, 128: padding to D + 8 gives (a) but puts rows r and r + 2 of (b)
// on 8 common banks.  shift is linear over row bases that are multiples of 4:
// off(r0 + x) = off(r0) + off(x) for r0 % 4 == 0, which keeps fragment offsets immediate.
static constexpr int RAGGED = -1;  // RowTile LDR value selecting this layout
template <int D>
struct Ragged {
  static_assert(D == 32 || D == 64 || D == 128, "head dims 32, 64, 128");
  __host__ __device__ static constexpr int shift(int r) {
    return D == 32 ? (r >> 2) : D == 64 ? 5 * (r >> 2) + 4 * ((r >> 1) & 1) : 13 * (r >> 2) + 4 * (r & 3);
  }
  __host__ __device__ static constexpr int off(int r) { return r * D + 8 * shift(r); }
  __host__ __device__ static constexpr int elems(int rows) { return off(rows - 1) + D; }
};

// Register-staged tiles for software pipelining: init() fixes each thread's byte offsets once,
// load() issues the global reads of a tile into registers (rows >= nvalid read as zero),
// store() writes them to LDS later.
template <typename T, int ROWS, int D, int LDR, int NT = 256>
struct RowTile {
  static constexpr int EPV = 16 / sizeof(T);
  static constexpr int CPR = D / EPV;
  static constexpr int NCH = ROWS * CPR;
  static constexpr int PER = (NCH + NT - 1) / NT;
  uint4 r[PER];
  uint32_t off[PER];
  __device__ __forceinline__ void init(int64_t ld, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + NT * i;
      const int row = c / CPR, col = (c % CPR) * EPV;
      off[i] = (uint32_t)(((int64_t)row * ld + col) * sizeof(T));
    }
  }
  __device__ __forceinline__ void load(const T* __restrict__ g, int64_t ld, int nvalid, int tid) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(g, tile_bytes<T, D>(ld, min(nvalid, ROWS)));
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (NCH % NT == 0 || tid + NT * i < NCH) r[i] = buf_load16(rs, off[i]);
  }
  __device__ __forceinline__ void store(T* __restrict__ lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + NT * i;
      const int row = c / CPR, col = (c % CPR) * EPV;
      if constexpr (LDR == RAGGED) {
        // row = tid / CPR + i * (NT / CPR), the second part a multiple of 4 (linear in off)
        static_assert((NT / CPR) % 4 == 0 && NT % CPR == 0, "ragged tile store");
        if (NCH % NT == 0 || c < NCH)
          *reinterpret_cast<uint4*>(lds + Ragged<D>::off(tid / CPR) + Ragged<D>::off(i * (NT / CPR)) + col) = r[i];
      } else {
        if (NCH % NT == 0 || c < NCH) *reinterpret_cast<uint4*>(lds + row * LDR + col) = r[i];
      }
    }
  }
};

// Same, stored transposed as [D][ROWS] (row stride LDT).  16-bit types move two source rows
// per thread so every LDS write is one packed 32-bit (row, row+1) pair (one v_perm_b32 each).
// For 16-bit types the rows of every group of 16 are stored in the order 0-3, 8-11, 4-7,
// 12-15 (bits 2 and 3 of the row index swapped): the 8 rows one MFMA fragment pairs with
// accumulator registers (row_of) are then contiguous and load_perm_frag reads them with a
// single 16-byte access.
template <typename T, int ROWS, int D, int LDT, int NT = 256>
struct TransTile {
  static constexpr int EPV = 16 / sizeof(T);
  static constexpr int CPR = D / EPV;
  static constexpr bool PAIR = sizeof(T) == 2;
  static constexpr int NU = PAIR ? (ROWS / 2) * CPR : ROWS * CPR;
  static constexpr int PER = (NU + NT - 1) / NT;
  uint4 r0[PER], r1[PAIR ? PER : 1];
  uint32_t off[PER];
  __device__ __forceinline__ void init(int64_t ld, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + NT * i;
      int row, col;
      if constexpr (PAIR) {
        row = 2 * (u % (ROWS / 2));
        col = (u / (ROWS / 2)) * EPV;
      } else {
        row = u % ROWS;
        col = (u / ROWS) * EPV;
      }
      off[i] = (uint32_t)(((int64_t)row * ld + col) * sizeof(T));
    }
  }
  __device__ __forceinline__ void load(const T* __restrict__ g, int64_t ld, int nvalid, int tid) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(g, tile_bytes<T, D>(ld, min(nvalid, ROWS)));
    const uint32_t step = (uint32_t)(ld * sizeof(T));
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (NU % NT != 0 && tid + NT * i >= NU) continue;
      r0[i] = buf_load16(rs, off[i]);
      if constexpr (PAIR) r1[i] = buf_load16(rs, off[i] + step);
    }
  }
  __device__ __forceinline__ void store(T* __restrict__ lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + NT * i;
      if (NU % NT != 0 && u >= NU) continue;
      if constexpr (PAIR) {
        const int kp = u % (ROWS / 2), col = (u / (ROWS / 2)) * EPV;
        const int k = 2 * kp, pos = (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
        const uint32_t a4[4] = {r0[i].x, r0[i].y, r0[i].z, r0[i].w};
        const uint32_t b4[4] = {r1[i].x, r1[i].y, r1[i].z, r1[i].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          *reinterpret_cast<uint32_t*>(lds + (col + 2 * e) * LDT + pos) = __builtin_amdgcn_perm(b4[e], a4[e], 0x05040100u);
          *reinterpret_cast<uint32_t*>(lds + (col + 2 * e + 1) * LDT + pos) = __builtin_amdgcn_perm(b4[e], a4[e], 0x07060302u);
        }
      } else {
        const int row = u % ROWS, col = (u / ROWS) * EPV;
        const float v[4] = {__uint_as_float(r0[i].x), __uint_as_float(r0[i].y), __uint_as_float(r0[i].z),
                            __uint_as_float(r0[i].w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) reinterpret_cast<float*>(lds)[(col + e) * LDT + row] = v[e];
      }
    }
  }
};

// A fragment whose contraction index runs along a contiguous LDS row, with the k slots
// paired to accumulator registers (row_of mapping).  `row` points at the first key of a
// 32-key block; j is the instruction index inside the block.
template <int DT>
__device__ __forceinline__ typename Tr<DT>::frag load_perm_frag(const typename Tr<DT>::T* row, int j, int g) {
  typedef typename Tr<DT>::frag frag;
  if constexpr (Tr<DT>::KPL == 8) {
    // rows 16j+4g+(0..3) and 16j+8+4g+(0..3), stored contiguously by TransTile
    return __builtin_bit_cast(frag, *reinterpret_cast<const uint4*>(row + 16 * j + 8 * g));
  } else {
    return row[row_of(j, g)];
  }
}

// The same fragment as load_perm_frag over a transposed tile, read instead from the row-major
// [rows][ldr] tile with gfx950's transposing LDS read (16-bit types): in each group of 16 lanes,
// lane a + 4m supplies the address of 4 consecutive columns of one row, and lane 4a + b receives
// column b of the rows supplied by lanes a, a+4, a+8, a+12.  Here lane a + 4m of group G points
// at row row0 + 16j + 4g + m (then + 8), columns col0 + 16 (G & 1) + 4a, so lane l receives column
// col0 + l % 32 of rows row0 + 16j + 4g + (0..3) and row0 + 16j + 8 + 4g + (0..3) (g = l / 32):
// the k slots of load_perm_frag / row_of.  No transposed copy of the tile is stored.
typedef short s16x4 __attribute__((ext_vector_type(4)));
template <int DT>
__device__ __forceinline__ typename Tr<DT>::frag load_tr_frag(const typename Tr<DT>::T* tile, int ldr, int row0, int col0,
                                                              int j, int lane) {
  static_assert(Tr<DT>::KPL == 8, "16-bit types only");
  const int G = lane >> 4, i = lane & 15, g = lane >> 5;
  const typename Tr<DT>::T* p = tile + (row0 + 16 * j + 4 * g + (i >> 2)) * ldr + col0 + 16 * (G & 1) + 4 * (i & 3);
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 8 * ldr));
  const uint2 xu = __builtin_bit_cast(uint2, x), yu = __builtin_bit_cast(uint2, y);
  return __builtin_bit_cast(typename Tr<DT>::frag, make_uint4(xu.x, xu.y, yu.x, yu.y));
}

// Element offset of row r in a row-major tile of row stride LDR, or of the ragged layout.
template <int LDR, int D>
__device__ __forceinline__ constexpr int row_off(int r) {
  if constexpr (LDR == RAGGED) return Ragged<D>::off(r);
  else return r * LDR;
}

// load_tr_frag over a tile of layout LDR (a stride or RAGGED); row0 a multiple of 16.
template <int DT, int LDR, int D>
__device__ __forceinline__ typename Tr<DT>::frag load_tr_frag_l(const typename Tr<DT>::T* tile, int row0, int col0, int j,
                                                                int lane) {
  static_assert(Tr<DT>::KPL == 8, "16-bit types only");
  const int G = lane >> 4, i = lane & 15, g = lane >> 5;
  const typename Tr<DT>::T* p =
      tile + row_off<LDR, D>(row0 + 16 * j) + row_off<LDR, D>(4 * g + (i >> 2)) + col0 + 16 * (G & 1) + 4 * (i & 3);
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + row_off<LDR, D>(8)));
  const uint2 xu = __builtin_bit_cast(uint2, x), yu = __builtin_bit_cast(uint2, y);
  return __builtin_bit_cast(typename Tr<DT>::frag, make_uint4(xu.x, xu.y, yu.x, yu.y));
}

// B fragment from accumulator values (registers j*KPL .. j*KPL+KPL-1).
template <int DT>
__device__ __forceinline__ typename Tr<DT>::frag acc_frag(const f32x16& a, int j) {
  typename Tr<DT>::frag f;
#pragma unroll
  for (int e = 0; e < Tr<DT>::KPL; ++e) Tr<DT>::set(f, e, a[j * Tr<DT>::KPL + e]);
  return f;
}

// Store a transposed accumulator block (lane = row `row`, registers = 16 columns of a
// 32-wide column block `d`) into a row-major [.., D] T tensor, scaled.
template <int DT>
__device__ __forceinline__ void store_acc_row(typename Tr<DT>::T* rowp, const f32x16& acc, int dblk, int g, float sc) {
  typedef typename Tr<DT>::T T;
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) {
    const int d0 = dblk * 32 + 8 * r4 + 4 * g;
    if constexpr (sizeof(T) == 2) {
      uint32_t w0 = (uint32_t)Tr<DT>::from_f(acc[4 * r4] * sc) | ((uint32_t)Tr<DT>::from_f(acc[4 * r4 + 1] * sc) << 16);
      uint32_t w1 = (uint32_t)Tr<DT>::from_f(acc[4 * r4 + 2] * sc) | ((uint32_t)Tr<DT>::from_f(acc[4 * r4 + 3] * sc) << 16);
      *reinterpret_cast<uint2*>(rowp + d0) = make_uint2(w0, w1);
    } else {
      *reinterpret_cast<float4*>(rowp + d0) =
          make_float4(acc[4 * r4] * sc, acc[4 * r4 + 1] * sc, acc[4 * r4 + 2] * sc, acc[4 * r4 + 3] * sc);
    }
  }
}

// LDS available to one workgroup on gfx950, and the waves-per-SIMD target of the main
// kernels (16-bit inputs fit two workgroups per CU; fp32 tiles need the whole register file).
static constexpr int LDS_LIMIT = 160 * 1024;

// Row padding (elements) of LDS tiles stored transposed ([D][64]) and read back with
// load_perm_frag: 16-byte reads per lane for 16-bit types, so rows stay 16-byte aligned
// (a 36-dword stride puts 8 consecutive rows of one read on distinct banks); fp32 reads are
// 4 bytes per lane from 32 rows, and a 65-dword stride spreads those over the banks.
template <typename T>
struct TransPad {
  static constexpr int value = sizeof(T) == 2 ? 8 : 1;
};
template <int DT>
struct Occ {
  static constexpr int value = DT == F32 ? 1 : 2;
};

struct Tensor4 {
  void* data;
  int64_t sb, sh, sl;  // element strides of the B, H, L dims; the D dim is contiguous
};

}  // namespace fla
