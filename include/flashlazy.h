/*
 * flashlazy.h -- C ABI of the MI355X (gfx950) AdaSplash / Lazy-Attention kernels.
 *
 * Every entry point takes raw device pointers, sizes and element strides, allocates
 * nothing, launches asynchronously on the caller's HIP stream (passed as `void*`,
 * a hipStream_t; NULL = default stream) and returns 0 on success, a negative
 * FLA_E* code for rejected arguments, or a positive hipError_t from the launch.
 *
 * Tensors of shape [B, H, L, D] are described by fla_tensor4_t: a data pointer and
 * the element strides of the B, H and L dimensions; the D dimension must be
 * contiguous, rows must be 16-byte aligned and 0 < stride_l * element size <= 16 MiB.  dtype is one of FLA_F32, FLA_F16,
 * FLA_BF16; D must be 32, 64 or 128 (callers pad smaller head dims with zeros and
 * pass the softmax scale of the true head dim).
 *
 * Attention entry points take H query heads and Hkv key/value heads (H % Hkv == 0):
 * query head h reads K/V head h / (H / Hkv) in place (grouped-query attention without a
 * repeat_interleave copy); k, v, dk, dv have Hkv heads, everything per row has H.  Hkv = H
 * is ordinary multi-head attention.
 */
#ifndef FLASHLAZY_H
#define FLASHLAZY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLA_OK 0
#define FLA_EINVAL (-1)
#define FLA_EUNSUPPORTED (-2)
#define FLA_EWORKSPACE (-3)

enum { FLA_F32 = 0, FLA_F16 = 1, FLA_BF16 = 2 };

typedef struct {
  void* data;
  int64_t stride_b, stride_h, stride_l;
} fla_tensor4_t;

/* Library version string. */
const char* fla_version(void);

/* Row-wise alpha-entmax over the last dimension of a [rows, n] matrix (row strides
 * ldx / ldy in elements).  Replaces the kernel behind
 * `adasplash.triton_entmax(x, alpha, n_iter, fast_math)` (reference README.md:28-35;
 * tests/test_triton_entmax.py).  1 < alpha <= 2.  The threshold is solved to fp32
 * convergence; n_iter only raises the iteration cap. */
int fla_entmax_fwd(const void* x, void* y, int64_t rows, int64_t n, int64_t ldx, int64_t ldy, int dtype, float alpha,
                   int n_iter, int fast_math, void* stream);

/* Backward of fla_entmax_fwd given its output y: dx = U dy - (sum U dy / sum U) U,
 * U = y^(2-alpha) on y > 0 (autograd backward of `triton_entmax`, gradcheck at
 * tests/test_triton_entmax.py:33-41). */
int fla_entmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t n, int64_t ldy, int64_t lddy,
                   int64_t lddx, int dtype, float alpha, void* stream);

/* Number of uint32 words per query-tile row of the AdaSplash block mask
 * (ceil(ceil(L/64)/32)).  The mask is [B, H, ceil(L/128), words]: bit c%32 of word
 * c/32 in row r is set iff some query i < varlen of tile r (rows 128r..128r+127) has
 * p_ij > 0 for a key j of tile c (keys 64c..64c+63). */
int fla_adasplash_mask_words(int L);

/* Expands a bit-packed block mask (rows of mw uint32 words; bit c%32 of word c/32 = column c,
 * as written by fla_adasplash_fwd / fla_lazy_fwd) into bytes: out[r * ncols + c] = bit c of
 * row r (0 or 1), ncols <= 32 * mw, in one launch on the caller's stream.  It yields the
 * boolean BMASK[b, h, m_block, n_block] of `lazy_attention_triton(..., return_mask=True)`
 * (reference CURSOR_TASKS.md:240-255, 283-286). */
int fla_unpack_block_mask(const uint32_t* words, uint8_t* out, int64_t rows, int mw, int ncols, void* stream);

/* AdaSplash forward: out = entmax_alpha(q k^T * scale, masked) v.
 * Replaces `adasplash(q, k, v, alpha, niter, is_causal, varlen)` (block-masked,
 * skip_empty_blocks = 1, block_mask written) and `adasplash_no_block_mask(...)`
 * (skip_empty_blocks = 0, block_mask may be NULL) -- reference README.md:39-58,
 * tests/test_adasplash.py, tests/test_adasplash_no_block_mask.py.
 *   tau  [B, H, L] fp32 out: threshold in (alpha-1)*score units, +inf on rows >= varlen.
 *   wn   [B, H, L, D] fp32 out, optional (needed by the backward):
 *        sum_j U_ij v_j / sum_j U_ij with U = p^(2-alpha).
 *   varlen [B] int32, optional: keys j >= varlen[b] are masked, output rows >= varlen[b] are zero.
 * niter is accepted for signature compatibility; the threshold is solved to fp32
 * convergence (niter raises the cap of the full-sweep fallback). */
int fla_adasplash_fwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                      const fla_tensor4_t* out, float* tau, float* wn, uint32_t* block_mask, const int32_t* varlen,
                      int B, int H, int Hkv, int L, int D, int dtype, float alpha, int niter, int is_causal,
                      int skip_empty_blocks, float scale, void* stream);

/* AdaSplash backward (dq, dk, dv) through the entmax Jacobian, from the forward's
 * tau and wn.  block_mask (optional) makes both backward kernels skip empty tiles.
 * delta_ws: caller-provided [B, H, L] fp32 scratch. */
int fla_adasplash_bwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                      const fla_tensor4_t* dout, const fla_tensor4_t* dq, const fla_tensor4_t* dk,
                      const fla_tensor4_t* dv, const float* tau, const float* wn, const uint32_t* block_mask,
                      const int32_t* varlen, float* delta_ws, int B, int H, int Hkv, int L, int D, int dtype, float alpha,
                      int is_causal, float scale, void* stream);

/* Lazy attention forward: causal elastic softmax relu(softmax(q k^T*scale + bias) + tau_h/(i+1)) v
 * with bias[h, i-j] added for 0 <= i-j < window.  Replaces `lazy_attention_triton`'s
 * forward (reference lazy_attention_triton.py:503-515, 543-583; kernels :9-174).
 *   bias fp32 [H, >= window] with row stride bias_ld; tau fp32 [H].
 *   lse [B, H, L] fp32 out: log-sum-exp of the scores in base-2 units, log2 sum_j 2^(s_ij log2 e)
 *        (= natural-log LSE * log2 e), the form fla_lazy_bwd consumes; +inf on rows >= varlen.
 *   wdelta [B, H, L, D] fp32 out, optional (needed by the backward):
 *          sum_j 1[p_ij + tau/(i+1) > 0] p_ij v_j.
 *   block_mask [B, H, ceil(L/64), fla_adasplash_mask_words(L)] uint32 out, optional: bit c%32
 *          of word c/32 in row r is set iff some e_ij = relu(p_ij + tau/(i+1)) > 0 with i in rows
 *          64r..64r+63 (i < varlen), j in keys 64c..64c+63 (j <= i, j < varlen) -- the planned
 *          block sparsity of CURSOR_TASKS.md:214-312 (BLOCK_M = BLOCK_N = 64).
 *   block_mask_u8 [B, H, ceil(L/64), ceil(L/64)] uint8 out, optional: the same blocks, one byte
 *          (0 / 1) each -- the boolean mask of `return_mask=True`, written by the forward itself.
 *   skip_empty_blocks: skip the P V / wdelta products of all-zero tiles (results unchanged).
 *          The backward cannot skip them: dS = p (m dP - delta) is non-zero where e = 0.
 *   varlen [B] int32, optional. */
int fla_lazy_fwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v, const fla_tensor4_t* out,
                 const float* bias, int64_t bias_ld, const float* tau, int window, float* lse, float* wdelta,
                 uint32_t* block_mask, uint8_t* block_mask_u8, int skip_empty_blocks, const int32_t* varlen, int B,
                 int H, int Hkv, int L, int D, int dtype, float scale, void* stream);

/* Bytes of caller-provided scratch that fla_lazy_bwd needs (per-tile dbias / dtau partials). */
size_t fla_lazy_bwd_workspace_size(int B, int H, int L, int window);

/* Lazy attention backward (reference lazy_attention_triton.py:518-541, 585-745; kernels :180-497).
 * dbias fp32 [H, window] and dtau fp32 [H] are optional (NULL = frozen parameters, the
 * reference's `_lazy_attention_backward_fast` path). */
int fla_lazy_bwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v, const fla_tensor4_t* dout,
                 const fla_tensor4_t* dq, const fla_tensor4_t* dk, const fla_tensor4_t* dv, const float* bias,
                 int64_t bias_ld, const float* tau, int window, const float* lse, const float* wdelta,
                 const int32_t* varlen, float* dbias, float* dtau, void* workspace, size_t workspace_bytes, int B,
                 int H, int Hkv, int L, int D, int dtype, float scale, void* stream);

/* Bytes of caller-provided scratch for fla_lazy_decode_fwd (0 for invalid sizes): per key chunk
 * partials and, for 16-bit inputs with fewer than D/4 query rows per K/V head, an fp32 cache of
 * the scores (rows x Lk).  The size does not depend on the dtype.  256-byte aligned. */
size_t fla_lazy_decode_workspace_size(int B, int H, int Hkv, int Lq, int Lk, int D);

/* Lazy attention over a KV cache (inference forward; decode and chunked prefill).  q, out are
 * [B, H, Lq, D]; k, v are the cache [B, Hkv, Lk, D].  Query i of batch b sits at position
 * pos = len_b - Lq + i (len_b = varlen[b] if given, else Lk) and attends to keys j <= pos,
 * j < len_b with the weights of fla_lazy_fwd at that position: relu(softmax(s + bias[h, pos-j]
 * for 0 <= pos-j < window) + tau_h/(pos+1)).  Rows with pos < 0 are zero.  This is the call the
 * reference's layer makes with a cache (examples/lazy_attention_layer.py:133-169), which its
 * square kernel (Lq = Lk assumed) does not cover.  No lse / backward state is produced. */
int fla_lazy_decode_fwd(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                        const fla_tensor4_t* out, const float* bias, int64_t bias_ld, const float* tau, int window,
                        const int32_t* varlen, void* workspace, size_t workspace_bytes, int B, int H, int Hkv, int Lq,
                        int Lk, int D, int dtype, float scale, void* stream);

/* Bytes of the static per-GPU scratch behind fla_lazy_decode_fwd_static (64 MiB). */
#define FLA_STATIC_SCRATCH_BYTES ((size_t)64 << 20)

/* fla_lazy_decode_fwd without a workspace argument.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  It calls no allocator; its scratch is a static device array
 * of FLA_STATIC_SCRATCH_BYTES that every GPU the library runs on holds until the process ends.
 * Returns FLA_EWORKSPACE when fla_lazy_decode_workspace_size(B, H, Hkv, Lq, Lk, D) exceeds that
 * size (use fla_lazy_decode_fwd there).  All calls on one GPU share its scratch: calls that
 * overlap in time on one GPU (e.g. on two streams) race and must be serialised by the caller.
 * Results are those of fla_lazy_decode_fwd. */
int fla_lazy_decode_fwd_static(const fla_tensor4_t* q, const fla_tensor4_t* k, const fla_tensor4_t* v,
                               const fla_tensor4_t* out, const float* bias, int64_t bias_ld, const float* tau,
                               int window, const int32_t* varlen, int B, int H, int Hkv, int Lq, int Lk, int D,
                               int dtype, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHLAZY_H */
