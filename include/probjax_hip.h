/*
 * probjax_hip.h -- C ABI of the MI355X (gfx950) fused-attention kernels that
 * back probjax.nn's attention path.
 *
 * Plain pointers and sizes only: every pointer is a device pointer into HBM
 * owned by the caller (XLA, torch, or a ctypes harness), valid for the
 * duration of the call; nothing is cached across calls.  `stream` is a
 * hipStream_t passed as void* (NULL = the default stream).  Every entry point
 * only enqueues work on `stream`: no device synchronisation, no host<->device
 * copies, no allocation.  Entry points are reentrant; the global state is a
 * thread-local error string, plus, for pjx_splitkv_decode_static only, one
 * library-held device array per GPU and its looked-up address.
 *
 * Layout conventions are probjax's: q [B, Lq, Hq, D], k/v [B, Lk, Hkv, D]
 * row-major (D fastest), query head h uses KV head h / (Hq / Hkv)
 * (probjax/nn/pallas_kernels/kernels/attention.py:2164-2165,2189-2196).
 *
 * Zero sizes: a tensor with no elements may be passed as a null pointer.  A
 * batch or query length of 0 computes nothing; a key / cache length of 0
 * gives every row output 0 and LSE +inf (the reference's rule for rows with
 * no valid key, attention_xla.py), and in the backward dq = 0 (no keys) or
 * dk = dv = 0 / dcache = 0 (no queries).
 *
 * Return value: PJX_OK, or an error code with a message in pjx_last_error().
 */
#ifndef PROBJAX_HIP_H_
#define PROBJAX_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of q, k, v, o (and cache / weights).  The bf16 and fp16
 * paths are the same kernels (v_mfma_f32_*_bf16 / _f16 operands, fp32
 * accumulation); P and dS are rounded to the input's 16-bit type before their
 * products, as the reference's casts to V's / Q's dtype do.  The reference's
 * fused paths take all three (layers/attention.py:1187,
 * kernels/attention.py:2678). */
#define PJX_DTYPE_F32 0
#define PJX_DTYPE_BF16 1
#define PJX_DTYPE_F16 2

#define PJX_OK 0
#define PJX_ERR_INVALID 1  /* unsupported shape / dtype / argument */
#define PJX_ERR_LAUNCH 2   /* the HIP runtime rejected a launch */
#define PJX_ERR_WORKSPACE 3 /* workspace missing or too small */

/*
 * Extended masks and score modifiers of pjx_flash_fwd / pjx_flash_bwd
 * (probjax/nn/pallas_kernels/attention_mask_bias.py).  Pass NULL for none;
 * in a struct, window_left / window_right < 0 and NULL pointers mean absent.
 * All device pointers; lengths and ids int32.
 *
 * Masks (ANDed with causal, kv_lengths and q_valid / kv_valid):
 *   causal_shift   -- with causal != 0, key k is visible to query q iff
 *                     k <= q + causal_shift: 0 for CausalMask (:617-648),
 *                     Lk - Lq for CausalFromBottomRightMask (:753-782)
 *   window_left    -- k >= q - window_left  (LocalWindowMask :651-704,
 *   window_right   -- k <= q + window_right  CausalLocalWindowMask :707-750)
 *   prefix_lengths -- [B]: k < P[b] or k <= q (PrefixLMMask :785-868)
 *   seq_lengths    -- [B]: (q < L[b] and k < L[b]) or q == k (SeqLenMask
 *                     :1239-1398)
 *   segment_q, segment_k -- [B, Lq], [B, Lk]: ids equal (SameSegmentMask
 *                     :1537-1668, BlockDiagonalMask :871-981; with causal
 *                     BlockDiagonalCausalMask :984-1076)
 *   row_kv_lengths -- [B, Lq]: k < row_kv_lengths[b, q] (KeyPaddingMask
 *                     :1132-1236, whose payload the reference reads per query
 *                     row: get_data :1192-1204 with the query block spec
 *                     :1175-1190); excludes segment_q / segment_k
 * Score modifiers, on s = sm_scale * q.k in the order of SumBias (:553-582):
 *   s' = f(s) + bias + alibi + constant, with
 *   f(s) = softcap * tanh(s / softcap) if softcap > 0 (SoftCappingBias
 *          :2564-2603), else s * head_scales[h] if head_scales is given
 *          (PerHeadScaleBias :2606-2648), else s;
 *   alibi = -alibi_slopes[h] * (alibi_symmetric ? |q - k| : max(q - k, 0))
 *          (CausalAlibiBias :2230-2255, SymmetricAlibiBias :2355-2380,
 *          DistanceDecayBias :2387-2414; slopes [Hq]);
 *   constant (ConstantBias :1781-1805).
 * The backward multiplies dS by f'(s).  softcap and head_scales exclude each
 * other.
 */
typedef struct pjx_score_mods {
  int32_t causal_shift;
  int32_t window_left;
  int32_t window_right;
  const int32_t* prefix_lengths;
  const int32_t* seq_lengths;
  const int32_t* segment_q;
  const int32_t* segment_k;
  const float* alibi_slopes;
  int32_t alibi_symmetric;
  float softcap;
  const float* head_scales;
  float constant;
  const int32_t* row_kv_lengths;
} pjx_score_mods;

/* Library version (major*10000 + minor*100 + patch). */
int pjx_version(void);

/* Message of the last error on the calling thread ("" if none). */
const char* pjx_last_error(void);

/*
 * Kernel instances that the calling thread's last entry-point call launched,
 * in launch order, ';'-separated ("" if none), e.g.
 * "flash_bwd_dq_kernel<Bf16Fmt, 128, 0, 0, 1>;flash_bwd_dkdv_kernel<...>".
 * Diagnostics (which kernel a launcher picked for a shape); no counterpart in
 * the reference, whose Pallas launch has one kernel per call.  Valid until the
 * thread's next entry-point call.
 */
const char* pjx_last_launches(void);

/*
 * Flash-attention forward.  Replaces the Pallas `mha_forward` kernel and its
 * launch (`_mha_impl_raw`, probjax/nn/pallas_kernels/kernels/attention.py:
 * 377-533, 2130-2278) for the masks/biases of the path, with the semantics of
 * the XLA reference (kernels/attention_xla.py:339-429):
 *
 *   s = sm_scale * q.k (fp32)  [+ bias[b|0, h|0, q, k]]  then masked -> -inf,
 *   o = softmax(s) . v with fp32 accumulation; P is rounded to bf16 / fp16
 *   before the P.V product with 16-bit inputs; rows without a valid key give 0.
 *
 * Masks (ANDed), all optional:
 *   causal      -- CausalMask, q >= k (attention_mask_bias.py:615-646)
 *   kv_lengths  -- KVLenMask, k < kv_lengths[b], int32 [B] (:1399-1532)
 *   q_valid / kv_valid -- QKVLengthMask static lengths (:1077-1127);
 *                  pass q_len / kv_len for none.
 * bias: DenseBias data, fp32 [bias_batch, bias_heads, Lq, Lk] with
 *   bias_batch in {1, B}, bias_heads in {1, Hq} (attention_mask_bias.py:
 *   1807-1922); NULL for none.
 * lse: optional fp32 [B, Hq, Lq] natural-log log-sum-exp of the scores
 *   (+inf for rows without a valid key, as attention_xla.py:420); NULL skips.
 *
 * mods: extended masks / score modifiers (pjx_score_mods) or NULL.
 *
 * dtype: PJX_DTYPE_BF16, PJX_DTYPE_F16 or PJX_DTYPE_F32 for q, k, v, o.  head_dim
 * in {64, 128, 256} (k and v share it; the reference's fused path takes
 * head_dim <= 256, layers/attention.py:1193-1195).  sm_scale must be > 0.
 */
int pjx_flash_fwd(int dtype, const void* q, const void* k, const void* v, void* o,
                  float* lse, const int32_t* kv_lengths, const float* bias,
                  int64_t bias_batch, int64_t bias_heads, int64_t batch, int64_t q_len,
                  int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                  int64_t q_valid, int64_t kv_valid, int causal, float sm_scale,
                  const pjx_score_mods* mods, void* stream);

/*
 * Bytes of workspace pjx_flash_bwd needs: two fp32 values per query row
 * (sm_scale * delta, delta = sum_d o*do, and the base-2 LSE),
 * 8 * batch * q_heads * q_len.
 */
size_t pjx_flash_bwd_workspace_size(int64_t batch, int64_t q_heads, int64_t q_len);

/*
 * Bytes of workspace with which pjx_flash_bwd keeps the rounded dS between
 * its kernels (the dS route), or 0 where the route does not exist: it exists
 * for 16-bit inputs at head_dim 256.  A call there without bias, dbias or
 * score modifiers (or modifiers that lower to none) whose workspace holds at
 * least this many bytes runs: delta; dK/dV, which also stores dS (2 bytes per
 * score, in 32-query x 16-key blocks); the dQ kernel, dQ = dS K as one
 * product per score, where the two-kernel route recomputes S and dP for dQ
 * (the three products of the reference's dQ scan,
 * kernels/attention.py:1089-1150, become one).  At head dim 256 the two
 * recomputed products cost more than storing and re-reading dS; at 64 and
 * 128 they cost less, and those head dims keep the two-kernel route.  Same
 * roundings as the two-kernel route.  Size: pjx_flash_bwd_workspace_size()
 * rounded up to 256 bytes, plus 2 * batch * q_heads * q_len' * kv_len' bytes,
 * q_len' and kv_len' rounded up to 64.
 */
size_t pjx_flash_bwd_ds_workspace_size(int dtype, int64_t batch, int64_t q_heads, int64_t q_len,
                                       int64_t kv_len, int64_t head_dim);

/*
 * Flash-attention backward: dq, dk, dv of pjx_flash_fwd's output.  Replaces
 * the Pallas backward of `mha` (probjax/nn/pallas_kernels/kernels/
 * attention.py: _preprocess_backward_kernel 853-867, mha_backward_kernel
 * 909-1160, _mha_backward_raw 3505-3560 with the GQA group sums 2123-2128):
 *
 *   delta = sum_d o*do;  p = exp(s - lse);  ds = p * (do.v^T - delta) * sm_scale
 *   dv = sum_q r(p)^T do,  dk = sum_q r(ds)^T q,  dq = sum_k r(ds) k
 *   (r: rounding to the 16-bit input type; none in fp32)
 *
 * with s the forward's score (sm_scale * q.k + bias, masked keys excluded)
 * and fp32 accumulation; dk/dv sum the query heads of each KV head's group.
 * dbias: NULL, or fp32 [B, Hq, Lq, Lk] that receives dL/d(bias) per query
 * head, P (dP - delta) for every score (the gradient the reference's dense
 * path gives a bias tensor, layers/attention.py:1293-1319; its kernel path's
 * custom VJP returns zeros instead, attention.py:3262-3263).  Needs bias; the
 * caller zero-fills it (fully masked tiles are not written) and sums it over
 * the dimensions the bias broadcasts.
 *
 * Arguments as pjx_flash_fwd, plus: o the forward output, dout [B, Lq, Hq, D]
 * the output gradient, lse the forward's natural-log LSE [B, Hq, Lq] (+inf
 * rows contribute nothing); dq [B, Lq, Hq, D], dk and dv [B, Lk, Hkv, D]
 * (fully written, zeros where no valid score reaches).  workspace: at least
 * pjx_flash_bwd_workspace_size(batch, q_heads, q_len) bytes.  mods: the
 * forward's (pjx_score_mods) or NULL.  A workspace of at least
 * pjx_flash_bwd_ds_workspace_size() bytes selects the dS route where it applies.
 * dtype: PJX_DTYPE_BF16, PJX_DTYPE_F16 or PJX_DTYPE_F32 (all fp32 products, no
 * roundings).  head_dim in {64, 128, 256}.
 */
int pjx_flash_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
                  const void* dout, const float* lse, void* dq, void* dk, void* dv,
                  float* dbias, void* workspace, size_t workspace_bytes, const int32_t* kv_lengths,
                  const float* bias, int64_t bias_batch, int64_t bias_heads, int64_t batch,
                  int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                  int64_t head_dim, int64_t q_valid, int64_t kv_valid, int causal,
                  float sm_scale, const pjx_score_mods* mods, void* stream);

/*
 * Bytes of workspace pjx_splitkv_decode / pjx_mla_decode need for these sizes
 * (partial outputs and log-sum-exp terms of every KV chunk).
 *   rows   -- query rows per (batch, kv head): (Hq/Hkv)*Lq for GQA decode,
 *             Lq*H for MLA (heads folded onto the query axis).
 *   groups -- kv heads (GQA decode) or 1 (MLA).
 *   v_dim  -- output head dim.
 */
size_t pjx_decode_workspace_size(int64_t batch, int64_t groups, int64_t rows,
                                 int64_t kv_len, int64_t v_dim, int64_t chunk);

/*
 * GQA split-KV decode.  Replaces `splitkv_forward` / `_splitkv_kernel` and the
 * XLA log-sum-exp merge (probjax/nn/pallas_kernels/kernels/attention_splitkv.py:
 * 43-250) and extends it with the per-sequence KVLenMask that the reference
 * routes to the regular forward (kernels/attention.py:2672-2675).
 *
 * dtype PJX_DTYPE_BF16, PJX_DTYPE_F16 or PJX_DTYPE_F32 (full fp32 products) for q, k, v, o:
 * q [B, Lq, Hq, D]; k [B, Lk, Hkv, D], v [B, Lk, Hkv, Dv] (Lk = KV capacity;
 * D = head_dim, Dv = v_dim, each 64, 128 or 256: the reference takes any D
 * and Dv, padded to the next power of two, attention_splitkv.py:155-172);
 * kv_lengths int32 [B] (NULL = all Lk valid); o [B, Lq, Hq, Dv];
 * lse optional fp32 [B, Hq, Lq], natural log (attention_splitkv.py:248-250).
 * The (Hq/Hkv)*Lq query rows of a KV head are packed row = g*Lq + t
 * (attention_splitkv.py:121-126), any number of them: up to 64 rows share one
 * pass over the keys (32 in fp32 or at D or Dv 256), more run as several row
 * groups, each streaming the keys (the reference's row blocks, :160-161).
 * Only keys < kv_lengths[b] are read.
 * chunk: keys per work item (0 = automatic: a power of two in [128, 2048]
 *   leaving about 1024 items at full capacity; else a multiple of 128).
 * workspace: at least pjx_decode_workspace_size(B, Hkv, rows, Lk, Dv, chunk) bytes.
 * Caches whose capacity B*Lk*Hkv*(D+Dv) exceeds 768 MiB of 16-bit data are
 * read with non-temporal loads (they do not fit the 256 MB MALL); smaller
 * ones with ordinary loads.  The environment variable PJX_DECODE_STREAM=0 or
 * =1 forces either; results are identical.
 */
int pjx_splitkv_decode(int dtype, const void* q, const void* k, const void* v,
                       const int32_t* kv_lengths, void* o, float* lse, void* workspace,
                       size_t workspace_bytes, int64_t batch, int64_t q_len,
                       int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                       int64_t head_dim, int64_t v_dim, float sm_scale, int64_t chunk, void* stream);

/*
 * Size of the library-held device array behind pjx_splitkv_decode_static:
 * 32 MiB on each GPU the library runs on, held until the process ends.
 */
#define PJX_DECODE_STATIC_SCRATCH_BYTES (32u << 20)

/*
 * pjx_splitkv_decode without a workspace argument: the partials go to the
 * library's own device array of PJX_DECODE_STATIC_SCRATCH_BYTES per GPU, and
 * nothing is allocated.  No counterpart in the reference: an extra entry for
 * callers that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Arguments, results and errors as
 * pjx_splitkv_decode (every argument is checked first); sizes whose partials
 * (pjx_decode_workspace_size(batch, kv_heads, rows, kv_len, v_dim, chunk))
 * exceed the array are then rejected with PJX_ERR_WORKSPACE.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (concurrent streams
 * or threads) race and must be serialised by the caller.
 */
int pjx_splitkv_decode_static(int dtype, const void* q, const void* k, const void* v,
                              const int32_t* kv_lengths, void* o, float* lse, int64_t batch,
                              int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                              int64_t head_dim, int64_t v_dim, float sm_scale, int64_t chunk,
                              void* stream);

/*
 * Latent (MLA) attention decode, absorbed form K = V = cache.  Replaces the
 * absorbed `mla_forward` kernel (probjax/nn/pallas_kernels/kernels/
 * latent_attention.py:79-197, 247-377, 636-766) with heads folded onto the
 * query axis (layers/latent_attention.py:458-469, row = t*H + h).
 *
 * q [B, Lq, H, R] and cache [B, S, R] of dtype (PJX_DTYPE_BF16 or PJX_DTYPE_F16);
 * kv_lengths int32 [B] or NULL;
 * o [B, Lq, H, v_dim] of dtype = the first v_dim columns of mla(q, cache, None,
 * None) (v_dim == R gives the API-exact output); lse optional fp32 [B, H, Lq].
 * (rank, v_dim) in {(576, 512), (576, 576), (512, 512), (256, 256), (128, 128),
 * (64, 64)}.  Any
 * Lq*H: each 16 folded rows form a row group that streams the cache chunk by
 * chunk (the reference's mla takes any head count, latent_attention.py:636-766).
 * chunk: keys per work item (0 = automatic, as for pjx_splitkv_decode; else a
 *   multiple of 64).
 * workspace: at least pjx_decode_workspace_size(B, 1, Lq*H, S, v_dim, chunk)
 * bytes with the same chunk.
 * Latents of more than 512 MiB (B*S*R 16-bit values) are read with
 * non-temporal loads, smaller ones with ordinary loads; PJX_DECODE_STREAM=0
 * or =1 forces either, with identical results.
 */
int pjx_mla_decode(int dtype, const void* q, const void* cache, const int32_t* kv_lengths,
                   void* o, float* lse, void* workspace, size_t workspace_bytes,
                   int64_t batch, int64_t q_len, int64_t heads, int64_t kv_len,
                   int64_t rank, int64_t v_dim, float sm_scale, int64_t chunk,
                   void* stream);

/*
 * Latent (MLA) attention forward, absorbed form K = V = cache, any query
 * length.  Replaces the absorbed `mla_forward` kernel and its launch
 * (probjax/nn/pallas_kernels/kernels/latent_attention.py: _mla_forward_kernel
 * 79-197 with wk = wv = None, _mla_build 247-377, mla_fwd_absorbed_p 380-388,
 * called from mla 636-766) with the masks and bias of pjx_flash_fwd:
 *
 *   s = sm_scale * q.c (fp32) [+ bias] then masked -> -inf;
 *   o = softmax(s) . c[:, :v_dim], P rounded to the 16-bit dtype before the product.
 *
 * q [B, Lq, H, R] (all H heads share the one latent head; folded calls
 * pass [B, Lq*H, 1, R] with H = 1); cache [B, S, R]; o [B, Lq, H, v_dim]
 * = the first v_dim columns of mla(q, cache, None, None) (v_dim == R
 * gives the API-exact output); lse optional fp32 [B, H, Lq] natural log.
 * kv_lengths, bias ([1|B, 1|H, Lq, S] fp32), q_valid / kv_valid, causal and
 * mods as for pjx_flash_fwd (with Lk = S, Hq = H).
 * (rank, v_dim) in {(576, 512), (576, 576), (512, 512)}, or rank in
 * {64, 128, 256} with v_dim == rank (the flash kernels with one K = V head).
 * dtype PJX_DTYPE_BF16 or PJX_DTYPE_F16 for q, cache, o.
 */
int pjx_mla_fwd(int dtype, const void* q, const void* cache, void* o, float* lse,
                const int32_t* kv_lengths, const float* bias, int64_t bias_batch,
                int64_t bias_heads, int64_t batch, int64_t q_len, int64_t kv_len,
                int64_t heads, int64_t rank, int64_t v_dim, int64_t q_valid, int64_t kv_valid,
                int causal, float sm_scale, const pjx_score_mods* mods, void* stream);

/*
 * Bytes of workspace pjx_mla_bwd needs for these sizes: sm_scale * delta and
 * the base-2 LSE per query row, plus fp32 partial cache gradients of the query-head
 * groups the key-side kernel splits the heads into (a function of the sizes
 * only).
 */
size_t pjx_mla_bwd_workspace_size(int64_t batch, int64_t heads, int64_t q_len, int64_t kv_len,
                                  int64_t rank);

/*
 * Backward of pjx_mla_fwd: dq and dcache.  Replaces the custom VJP of the
 * absorbed `mla` (probjax/nn/pallas_kernels/kernels/latent_attention.py:
 * 752-766), which differentiates the materialised computation: mha over
 * K = V = the latent broadcast to every head (_materialize_kv :396-410,
 * _materialized_mla :413-468), so that
 *
 *   delta = sum_d o*do;  p = exp(s - lse);  ds = p * (do.c[:, :v_dim]^T - delta) * sm_scale
 *   dq = sum_k r(ds) c,
 *   dcache = sum over heads and queries of r(ds)^T q + r(p)^T do (first v_dim dims)
 *   (r: rounding to the 16-bit dtype)
 *
 * with fp32 accumulation (the sum over heads in fp32 before one rounding).
 * The bias gets no gradient, as the reference's VJP returns none for mask
 * and bias leaves.  Arguments as pjx_mla_fwd, plus o (the forward output
 * [B, Lq, H, v_dim]), dout (its gradient, same shape), lse (the forward's
 * [B, H, Lq] natural-log LSE); dq [B, Lq, H, rank] and dcache [B, S, rank] are
 * fully written.  workspace: at least pjx_mla_bwd_workspace_size(batch, heads,
 * q_len, kv_len, rank) bytes.  (rank, v_dim) in {(576, 512), (576, 576),
 * (512, 512)}; dtype PJX_DTYPE_BF16 or PJX_DTYPE_F16.
 */
int pjx_mla_bwd(int dtype, const void* q, const void* cache, const void* o, const void* dout,
                const float* lse, void* dq, void* dcache, void* workspace, size_t workspace_bytes,
                const int32_t* kv_lengths, const float* bias, int64_t bias_batch,
                int64_t bias_heads, int64_t batch, int64_t q_len, int64_t kv_len, int64_t heads,
                int64_t rank, int64_t v_dim, int64_t q_valid, int64_t kv_valid, int causal,
                float sm_scale, const pjx_score_mods* mods, void* stream);

/*
 * Latent up-projection of materialised latent attention (mla with wk / wv).
 * Replaces the key/value formation of the reference: `_materialize_kv`
 * (probjax/nn/pallas_kernels/kernels/latent_attention.py:396-410) with the
 * zero head-dim padding of `_materialized_mla` (:413-468), the in-loop
 * `K = C W_K^T`, `V = C W_V^T` of `_mla_forward_kernel` (:132-177):
 *
 *   k[b, s, h, d] = sum_r cache[b, s, r] * wk[h, d, r]  (d < qk_dim; 0 up to width)
 *   v[b, s, h, d] = sum_r cache[b, s, r] * wv[h, d, r]  (d < v_dim;  0 up to width)
 *
 * fp32 accumulation, rounded to dtype (PJX_DTYPE_BF16, PJX_DTYPE_F16 or PJX_DTYPE_F32; all
 * operands the same dtype).  cache [B, S, R]; wk [H, qk_dim, R];
 * wv [H, v_dim, R]; k, v [B, S, H, width] fully written.  The flash kernels
 * then attend q (zero-padded to width) over k / v: the padded channels carry
 * zeros, so scores and the first v_dim output channels are unchanged.
 * 1 <= qk_dim, v_dim <= width; H * width <= 2^20.
 */
int pjx_mla_project(int dtype, const void* cache, const void* wk, const void* wv, void* k,
                    void* v, int64_t batch, int64_t kv_len, int64_t heads, int64_t rank,
                    int64_t qk_dim, int64_t v_dim, int64_t width, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PROBJAX_HIP_H_ */
