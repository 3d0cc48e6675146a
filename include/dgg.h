/*
 * dgg.h - C ABI of libdgg_hip.so, the MI355X (gfx950) kernels of the DeepGenGraph attention hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, sizes and element strides (no framework types),
 *   - never allocates or frees device memory (scratch is passed in by the caller),
 *   - validates every argument on the host before anything is launched,
 *   - launches asynchronously on the given hipStream_t (passed as void*; NULL = default stream),
 *   - returns DGG_OK (0) or a negative DGG_ERR_* code; the message of the last failure on the
 *     calling thread is returned by dgg_last_error().
 *
 * dtype codes follow the order of the reference's dispatch macro
 * (csrc/utils.h:3-8: Float, Half, BFloat16).
 */
#ifndef DGG_H_
#define DGG_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: dgg_ref_multiplier removed; DGG_ATTN_REF_ROUNDING divides as torch does on the GPU (multiply by the fp32
 * reciprocal); top-k ranks NaN above +inf; the split-KV entry points (dgg_attn_splitkv*) added. */
#define DGG_ABI_VERSION 2

enum dgg_dtype { DGG_F32 = 0, DGG_F16 = 1, DGG_BF16 = 2 };

enum dgg_status {
  DGG_OK = 0,
  DGG_ERR_DTYPE = -1,       /* dtype not supported by this op */
  DGG_ERR_SHAPE = -2,       /* a size is negative, zero where it must not be, or inconsistent */
  DGG_ERR_STRIDE = -3,      /* innermost stride is not 1, or a stride is not a multiple of the vector width */
  DGG_ERR_ALIGN = -4,       /* a pointer is not aligned to the vector width */
  DGG_ERR_UNSUPPORTED = -5, /* head_dim / option combination without a kernel */
  DGG_ERR_LAUNCH = -6,      /* hipGetLastError() reported a failure after the launch */
  DGG_ERR_NULL = -7,        /* a required pointer is NULL */
  DGG_ERR_WORKSPACE = -8    /* caller-provided scratch is too small */
};

/* Flags for the attention entry points. */
#define DGG_ATTN_CAUSAL 0x1u /* bottom-right aligned causal mask: key j is visible to query i iff j <= i + (Sk - Sq) */
/* Round scores to the input dtype at the points where the reference's eager module rounds them
 * (Q.K^T result, the 1/sqrt(D) scaling, each soft-cap step) before the fp32 softmax. Each division by a
 * Python float there is evaluated as torch does on the GPU: an fp32 multiply by the fp32 reciprocal of the
 * fp32 divisor (sqrt(D) for the default scale, else 1 / scale; the soft-cap), rounded to the dtype. Costs a
 * few VALU ops per score; used where downstream selection (H2O top-k) depends on exact probabilities. */
#define DGG_ATTN_REF_ROUNDING 0x2u
/* lse in base 2 (log2 of the row sum of 2^(scores*log2(e)), i.e. the natural lse times log2(e)):
 * dgg_attn_prefill writes it so and dgg_attn_colsum reads it so. Saves one multiply per score in the
 * column-sum pass when the caller only hands the lse from one to the other (as H2O does). */
#define DGG_ATTN_LSE_BASE2 0x4u

int dgg_abi_version(void);
const char* dgg_last_error(void);

/* ---------------------------------------------------------------------------------------------
 * Elementwise ops: replace the pybind11 module of csrc/ffi.cpp:4-8 (prototypes csrc/op.h:2-6).
 * Rows are [rows, hidden]; strides are in elements between consecutive rows; columns are contiguous.
 * ------------------------------------------------------------------------------------------- */

/* csrc/norm.cu:85-98 rms_norm(out, input, weight, epsilon):
 *   out[r,i] = T( T(x[r,i] * rsqrt(mean_i x[r,i]^2 + eps)) * w[i] ), fp32 accumulation.
 * weight has the input dtype (csrc/norm.cu:96). out may alias input. */
int dgg_rms_norm(void* out, const void* input, const void* weight, int64_t rows, int64_t hidden,
                 int64_t in_row_stride, int64_t out_row_stride, int dtype, float epsilon, void* stream);

/* csrc/norm.cu:100-113 fused_add_rms_norm(input, residual, weight, epsilon), in place:
 *   residual = T(input + residual);  input = rms_norm(residual).  (Not exported by the reference's
 *   ffi.cpp; provided for the Llama layer's residual + norm pair.) */
int dgg_fused_add_rms_norm(void* input, void* residual, const void* weight, int64_t rows, int64_t hidden,
                           int64_t in_row_stride, int64_t res_row_stride, int dtype, float epsilon,
                           void* stream);

/* csrc/activation.cu:24-34 silu_and_mul(out, input): input [rows, 2d] = [gate | up],
 *   out[r,i] = T( T(silu(gate[r,i])) * up[r,i] ). */
int dgg_silu_and_mul(void* out, const void* input, int64_t rows, int64_t d, int64_t in_row_stride,
                     int64_t out_row_stride, int dtype, void* stream);

/* dgg_rms_norm on [norm_rows, hidden] and dgg_silu_and_mul on [act_rows, 2d] in one launch (no counterpart as one
 * call in the reference: the two ops of the decode step's RmsNorm.forward and MLP.forward, llama_base.py:287-289,
 * 305-314, each csrc/norm.cu:85-98 and csrc/activation.cu:24-34). Results are those of the two calls; the one-launch
 * form needs 16-byte aligned rows (else the two kernels run one after the other). Either row count may be 0. */
int dgg_rms_norm_silu_and_mul(void* norm_out, const void* norm_in, const void* weight, int64_t norm_rows,
                              int64_t hidden, int64_t norm_in_row_stride, int64_t norm_out_row_stride, float epsilon,
                              void* act_out, const void* act_in, int64_t act_rows, int64_t d,
                              int64_t act_in_row_stride, int64_t act_out_row_stride, int dtype, void* stream);

/* csrc/pos_encoding.cu:180-199 rotary_embedding_online(positions, query, key, head_size, rope_theta):
 * NeoX pairing (i, i + D/2), angle = pos / theta^(2i/D) in fp32, in place on query [tokens, head_num*D]
 * and key [tokens, kv_head_num*D] with row strides q_row_stride / k_row_stride.
 * The reference asserts D == 128 (pos_encoding.cu:195); this build accepts any even D that is a
 * multiple of 16 up to 512 and returns DGG_ERR_UNSUPPORTED otherwise. key may be NULL (Q only). */
int dgg_rotary_embedding_online(const int32_t* positions, void* query, void* key, int64_t tokens,
                                int64_t head_num, int64_t kv_head_num, int64_t head_dim, int64_t q_row_stride,
                                int64_t k_row_stride, int dtype, float rope_theta, void* stream);
/* csrc/pos_encoding.cu:152-178 rotary_embedding(positions, query, key, head_size, cos_sin_cache, is_neox) (the kernel
 * of pos_encoding.cu:7-61; not exported by the reference's ffi.cpp): in place on query [tokens, head_num*head_size]
 * and key [tokens, kv_head_num*head_size] (row strides as dgg_rotary_embedding_online; key may be NULL), with
 * cos_sin_cache [max_position, rot_dim] of the input dtype, row p = [cos (rot_dim/2) | sin (rot_dim/2)]. is_neox:
 * pairs (i, i + rot_dim/2), else GPT-J pairs (2i, 2i+1), i < rot_dim/2; dims past rot_dim are untouched.
 * x' = x*cos - y*sin, y' = y*cos + x*sin with the reference's rounding: for f16/bf16 each product and the result are
 * rounded to the dtype (c10 Half / BFloat16 arithmetic). A token whose position lies outside [0, max_position) is
 * left unchanged (the reference would read outside the cache). rot_dim even, 2 <= rot_dim <= head_size. */
int dgg_rotary_embedding(const int32_t* positions, void* query, void* key, int64_t tokens, int64_t head_num,
                         int64_t kv_head_num, int64_t head_size, int64_t q_row_stride, int64_t k_row_stride,
                         const void* cos_sin_cache, int64_t rot_dim, int64_t max_position, int is_neox, int dtype,
                         void* stream);
/* The (cos, sin) table of the online rotary for dgg_attn_prefill_rope (no counterpart in the reference; the values
 * are those rotary_embedding_online computes, pos_encoding.cu:83-86): cos_sin fp32 [tokens, head_dim], row t =
 * cos(pos[t] / theta^(2i/head_dim)) for i < head_dim/2, then the sines. */
int dgg_rotary_cos_sin(const int32_t* positions, float* cos_sin, int64_t tokens, int64_t head_dim, float rope_theta,
                       void* stream);

/* ---------------------------------------------------------------------------------------------
 * Attention. The reference has no kernel ABI for attention: it is the callable returned by
 * compile(model, input_names, inputs, output_names, system) (compile.py:6,296) that runs
 * Attn.forward / Gemma2.forward / H2O.forward (deepgengraph_exp/cases/kernels/{attn,gemma2,h2o}.py).
 * These entry points are what that callable launches here.
 *
 * Layout: q [B, Sq, Hq, D], k/v [B, Sk, Hkv, D], o [B, Sq, Hq, D] (the case modules' layout), given as
 * element strides {batch, seq, head} with the D stride fixed at 1. Hq must be a multiple of Hkv
 * (query head h reads KV head h / (Hq/Hkv)). dtype: DGG_F16 or DGG_BF16. D in {64, 128, 256}.
 * ------------------------------------------------------------------------------------------- */

/* Fused online-softmax attention forward.
 *   scores = (q . k^T) * scale; if softcap > 0: scores = softcap * tanh(scores / softcap);
 *   mask (flags & DGG_ATTN_CAUSAL: key j visible iff j <= i + Sk - Sq; window > 0: also iff
 *   i + Sk - Sq - j < window); p = softmax_j(scores) in fp32; o = p . v.
 * lse (optional, may be NULL): fp32 [B, Hq, Sq] contiguous, natural-log log-sum-exp of the masked
 * scaled scores (base 2 with DGG_ATTN_LSE_BASE2); -inf for a row with no visible key (its o row is NaN, as the
 * reference's softmax of an all -inf row; with Sk == 0, o is 0, the reference's P.V over an empty key axis). strides: 12 int64 = q{b,s,h}, k{b,s,h}, v{b,s,h}, o{b,s,h}. */
int dgg_attn_prefill(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t Sq,
                     int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides, float scale,
                     float softcap, int64_t window, uint32_t flags, int dtype, void* stream);
/* dgg_attn_prefill with the query's rotary embedding fused into the kernel (no counterpart as one call in the
 * reference: it replaces rotary_embedding_online on the query, csrc/pos_encoding.cu:180-199 via models/attn.py:41,
 * followed by the attention). Row i of batch b of q is rotated by row b * Sq + i of q_cos_sin, fp32
 * [B * Sq, 128]: the cos of the 64 angles pos / theta^(2j/128) followed by their sines, as dgg_rotary_cos_sin
 * writes them; the rotated row is rounded to the input dtype before use, as the rotary op stores it. q itself is
 * not modified. head_dim 128 and f16 / bf16 only; q_cos_sin 32-byte aligned. Other arguments as dgg_attn_prefill. */
int dgg_attn_prefill_rope(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t Sq,
                          int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides, float scale,
                          float softcap, int64_t window, uint32_t flags, int dtype, const float* q_cos_sin,
                          void* stream);

/* H2O column sums (deepgengraph_exp/cases/kernels/h2o.py:35-36): colsum[b,h,j] = sum_i p[b,h,i,j] with p
 * the fp32 probabilities of dgg_attn_prefill, recomputed from q, k and the lse it wrote (same scale,
 * softcap, window and flags, DGG_ATTN_LSE_BASE2 included). colsum: fp32 [B, Hq, Sk] contiguous. strides: 6 int64 = q{b,s,h}, k{b,s,h}. */
int dgg_attn_colsum(const void* q, const void* k, const float* lse, float* colsum, int64_t B, int64_t Sq,
                    int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides, float scale,
                    float softcap, int64_t window, uint32_t flags, int dtype, void* stream);

/* Column-score epilogues of dgg_attn_colscore: the other KV-selection cases of the reference on the same
 * two-pass scheme (forward with lse, then column pass).
 *   DGG_COL_SUM:    out0[b,h,j] = sum_i p[b,h,i,j]                  (H2O h2o.py:35-36; SnapKV snapkv.py:36-37)
 *   DGG_COL_SUM_SQ: out0 = sum_i p, out1 = sum_i p^2                (RoCo roco.py:43-47)
 *   DGG_COL_ANY_GE: out_any[b,h,j] = any_i (p[b,h,i,j] >= thr[i*thr_row_stride + j]), uint8 0/1
 *                                                                   (Corm corm.py:35-37; thr = corm_mask [Sq, Sk])
 * Rows i >= Sq take no part. As in the reference, every query row is compared: a masked pair of a row that sees
 * at least one key has p = 0 (softmax of -inf), so it flags its key when thr <= 0; a row that sees no key at all
 * (Sq > Sk, causal) has NaN probabilities and flags nothing. DGG_COL_ANY_GE launches a second small kernel for the
 * masked pairs (it reads the masked part of thr once for all heads), and at head_dim 128 the column pass stops a
 * workgroup once all of its keys are flagged (an OR cannot change after that). The two new epilogues take no
 * soft-cap (DGG_ERR_UNSUPPORTED). Other arguments as dgg_attn_colsum. */
#define DGG_COL_SUM 0
#define DGG_COL_SUM_SQ 1
#define DGG_COL_ANY_GE 2
int dgg_attn_colscore(const void* q, const void* k, const float* lse, int epilogue, float* out0, float* out1,
                      uint8_t* out_any, const float* thr, int64_t thr_row_stride, int64_t B, int64_t Sq, int64_t Sk,
                      int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides, float scale, float softcap,
                      int64_t window, uint32_t flags, int dtype, void* stream);

/* KeyFormer (deepgengraph_exp/cases/kernels/kf.py:18-40), which sums over the queries the softmax of the
 * Gumbel-perturbed scores kf = softmax((scores + gumbels) / tau) with gumbels = -log(exp_rand) (kf.py:36-40):
 * two passes after the plain forward (dgg_attn_prefill gives the case's `out`).
 *   dgg_attn_kf_rowlse: lse2[b,h,i] = log2 sum_j exp((s[b,h,i,j] - ln exp_rand[b,h,i,j]) / tau) over the keys
 *     row i sees (-inf for a row that sees none); fp32 [B, Hq, Sq] contiguous, base 2.
 *   dgg_attn_kf_colsum: kf_score[b,h,j] = sum_i exp((s - ln exp_rand) / tau - lse2 ln 2), fp32 [B, Hq, Sk]
 *     contiguous, from the lse2 of the first pass.
 * s = q.k^T * scale as dgg_attn_prefill's scores (DGG_ATTN_REF_ROUNDING rounds them as the reference does,
 * kf.py:34), causal / window as there; no soft-cap. exp_rand: fp32 [B, Hq, Sq, Sk] with element strides
 * er_strides = {batch, head, row} and unit key stride, 4-byte aligned (16-byte aligned rows read faster);
 * values > 0. tau > 0. Sk >= 1. Other arguments as dgg_attn_colsum. The reference function replaced here is
 * the eager KeyFormer.forward; its compile()-produced callable is what deepgengraph_amd.compile returns. */
int dgg_attn_kf_rowlse(const void* q, const void* k, const float* exp_rand, const int64_t* er_strides, float* lse2,
                       int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides,
                       float scale, float tau, int64_t window, uint32_t flags, int dtype, void* stream);
int dgg_attn_kf_colsum(const void* q, const void* k, const float* exp_rand, const int64_t* er_strides,
                       const float* lse2, float* kf_score, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv,
                       int64_t D, const int64_t* strides, float scale, float tau, int64_t window, uint32_t flags,
                       int dtype, void* stream);

/* SnapKV pooling of the column sums (snapkv.py:38: F.avg_pool1d(kernel_size, padding = kernel_size // 2,
 * stride 1, count_include_pad)): out[r][j] = sum_{|t| <= kernel_size/2} in[r][j+t] / kernel_size with zeros
 * outside [0, n). in / out fp32 [rows, n] contiguous, not aliased; kernel_size odd. */
int dgg_avg_pool1d(const float* in, float* out, int64_t rows, int64_t n, int64_t kernel_size, void* stream);

/* KV-cache compaction after top-k (models/h2o.py:53-57, models/snapkv.py:54-57, models/kf.py:57-60):
 * out [B, 2, n_sel, Hkv, D] contiguous, out[b][0][i][h] = k[b][indices[b][h][i]][h], out[b][1][i][h] = v[...].
 * k / v are [B, S, Hkv, D] with element strides {batch, seq, head} (k then v: 6 int64); indices int64
 * [B, Hkv, n_sel] contiguous. An index outside [0, S) yields a zero row (nothing is read out of bounds).
 * Any dtype; rows of D elements must be a multiple of 16 bytes and 16-byte aligned. */
int dgg_kv_gather(const void* k, const void* v, const int64_t* indices, void* out, int64_t B, int64_t S, int64_t Hkv,
                  int64_t D, int64_t n_sel, const int64_t* strides, int dtype, void* stream);

/* Corm's selection of the flagged keys (deepgengraph_exp/cases/models/corm.py:53: torch.nonzero(corm_score)):
 * the coordinates of the nonzero bytes of a row-major tensor of shape dims[0..ndim), in row-major order, as
 * coords[i][0..ndim) int64 (the first min(total, max_out) entries are written). *total (device int64, 8-byte
 * aligned) receives the number of nonzeros. workspace: dgg_nonzero_workspace_bytes(rows) bytes, 8-byte aligned,
 * rows = numel / dims[ndim-1]. ndim in [1, 8]. Three launches; nothing is allocated. */
int64_t dgg_nonzero_workspace_bytes(int64_t rows);
int dgg_nonzero(const uint8_t* in, int ndim, const int64_t* dims, int64_t* coords, int64_t max_out, int64_t* total,
                void* workspace, int64_t workspace_bytes, void* stream);

/* Top-k of H2O scores (deepgengraph_exp/cases/models/h2o.py:51-52: torch.topk then sort of the indices):
 * for each of `rows` rows of n fp32 scores (row stride n), the k largest, ties broken by the lowest index,
 * written as int64 indices in ascending index order to out_idx [rows, k]. Values are ordered as torch.topk
 * orders them: -0.0 equals +0.0 and NaN (either sign) ranks above +inf. 1 <= k <= n <= 65536. */
int dgg_topk_indices(const float* scores, int64_t rows, int64_t n, int64_t k, int64_t* out_idx, void* stream);

/* dgg_topk_indices in either direction: largest != 0 is dgg_topk_indices; largest == 0 takes the k smallest
 * (torch.topk(..., largest=False), deepgengraph_exp/cases/models/roco.py:55), NaN last, ties again broken by the
 * lowest index. Output in ascending index order. */
int dgg_topk_select(const float* scores, int64_t rows, int64_t n, int64_t k, int largest, int64_t* out_idx,
                    void* stream);

/* RoCo's KV selection (deepgengraph_exp/cases/models/roco.py:54-61) for `rows` rows of n keys: from the column sums
 * score = roco_score and sq_score = roco_sq_score (fp32, row stride n), std = sqrt(sq_score / q_len -
 * (score / q_len) ** 2) rounded as torch computes it on the GPU (division by q_len = multiplication by the fp32
 * reciprocal, correctly rounded sqrt, NaN where cancellation makes the variance negative); recent = the `recent`
 * keys of largest std, other = the n - recent keys of smallest std, pick = the `budget` keys of other with the
 * largest score / q_len. out_idx [rows, budget + recent] receives pick and recent merged in ascending index order
 * (an index in both, possible only through ties, appears twice, as the reference's cat + sort keeps it). Ties are
 * broken by the lowest index in every selection. 0 <= recent <= n <= 65536, 0 <= budget <= n - recent. */
int dgg_roco_select(const float* score, const float* sq_score, int64_t rows, int64_t n, int64_t q_len, int64_t recent,
                    int64_t budget, int64_t* out_idx, void* stream);

/* Rows of more than 65536 keys (up to 2^26): dgg_topk_select and dgg_roco_select with the same results, computed
 * by many workgroups per row (a top-k with ceil(n / 8192) * k <= 65536 in two stages, a chunk-wise top-k and a
 * merge, reading the row once; others in radix passes; RoCo's `other` from the boundary of a two-stage `recent`,
 * in two reads of the row) through a caller-provided workspace of
 * dgg_select_workspace_bytes(rows, n) bytes (0 for n <= 65536, where these calls are dgg_topk_select /
 * dgg_roco_select and ignore the workspace), 256-byte aligned; rows <= 65535 when n > 65536. No counterpart in the
 * reference beyond the torch.topk calls they replace (models/h2o.py:51, models/snapkv.py:51, models/kf.py:54,
 * models/roco.py:54-61), which have no size limit. */
int64_t dgg_select_workspace_bytes(int64_t rows, int64_t n);
int dgg_topk_select_ws(const float* scores, int64_t rows, int64_t n, int64_t k, int largest, int64_t* out_idx,
                       void* workspace, int64_t workspace_bytes, void* stream);
int dgg_roco_select_ws(const float* score, const float* sq_score, int64_t rows, int64_t n, int64_t q_len,
                       int64_t recent, int64_t budget, int64_t* out_idx, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* Decode attention (Attn.forward with q_len == 1, attn.py:22-23: no mask) as split-KV + LSE merge.
 * q [B, Hq, D] strides {b,h}; k/v cache [B, Hkv, L, D] strides {b,h,l}; o [B, Hq, D] strides {b,h}.
 * strides: 10 int64 = q{b,h}, k{b,h,l}, v{b,h,l}, o{b,h}.
 * workspace: fp32 scratch of dgg_attn_decode_workspace_bytes(B, Hq, D, splits) bytes, 16B aligned:
 * per (b, h, split) the unnormalised partial output, its max and its sum.
 * lse (optional): fp32 [B, Hq], natural log. splits in [1, 1024]; L >= 1. */
int64_t dgg_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t D, int64_t splits);
int dgg_attn_decode(const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                    int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                    const int64_t* strides, int64_t splits, float scale, int dtype, void* stream);
/* Split-KV attention for a few query rows over a long key range. No kernel counterpart in the reference: it serves
 * the compile() callable of Attn / Gemma2 (attn.py:18-34, gemma2.py:19-38) when 1 <= q_len << kv_len, as in chunked
 * prefill, multi-row and speculative decode, and grouped-query decode. Semantics, layouts and the 12 strides are
 * those of dgg_attn_prefill (bottom-right causal mask, window, soft-cap, GQA, DGG_ATTN_LSE_BASE2); the lse is
 * written for every row. DGG_ATTN_REF_ROUNDING is not supported (DGG_ERR_UNSUPPORTED). The keys any row sees are cut
 * into `splits` slices; one workgroup takes a slice and up to 64 of the G * Sq rows of a KV head (its G = Hq / Hkv
 * query heads times the Sq query rows), so each K / V row is read once per 64 rows; a merge kernel combines the
 * slices. workspace: dgg_attn_splitkv_workspace_bytes(B, Sq, Hq, D, splits) bytes, 16-byte aligned. f16 / bf16,
 * Sq >= 1, Sk >= 1, splits in [1, 1024]. dgg_attn_decode and dgg_attn_decode_noalloc run grouped-query calls
 * (Hq > Hkv) through these kernels with the same workspace size. */
int64_t dgg_attn_splitkv_workspace_bytes(int64_t B, int64_t Sq, int64_t Hq, int64_t D, int64_t splits);
int dgg_attn_splitkv(const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                     int64_t workspace_bytes, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D,
                     const int64_t* strides, int64_t splits, float scale, float softcap, int64_t window,
                     uint32_t flags, int dtype, void* stream);
/* dgg_attn_decode without a workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc); no counterpart in the reference. The split
 * partials live in a fixed 96 MiB (100663296-byte) device array that each GPU the library runs on holds until the
 * process ends; a call whose partials, B * Hq * splits * (D + 2) * 4 bytes, exceed it returns
 * DGG_ERR_WORKSPACE. Nothing is allocated and nothing needs clearing between calls, but every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other threads) race. The stream must
 * belong to the current device. Arguments otherwise as dgg_attn_decode, with the same results. */
int dgg_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t Hq,
                            int64_t Hkv, int64_t L, int64_t D, const int64_t* strides, int64_t splits, float scale,
                            int dtype, void* stream);

/* Shader-clock probe (no counterpart in the reference: measurement support for the benchmark). One lane spins for
 * `ticks` ticks of the constant 100 MHz real-time counter and writes out[0] = shader cycles elapsed (s_memtime),
 * out[1] = real-time ticks elapsed: the shader clock is out[0] / out[1] * 100 MHz. out: 2 device uint64, 8-byte
 * aligned. ticks in [1, 10^6]. */
int dgg_clock_probe(unsigned long long* out, int64_t ticks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DGG_H_ */
