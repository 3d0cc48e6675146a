// Decode attention (one query token per sequence) as split-KV + log-sum-exp merge.
//
// Decode is HBM-bound: each (batch, head, split) workgroup streams its slice of the K and V caches once
// with 16-byte loads. Lanes are grouped D/8 per key row, so one wave instruction covers 512/D whole
// key rows (1 KiB contiguous per wave); the four waves of a workgroup interleave rows so that one
// iteration of the workgroup reads 2 KiB..4 KiB of contiguous cache. Each lane group keeps its own
// online-softmax state (max, sum, 8 output columns) in registers; the 4*512/D states of a workgroup are
// merged once through LDS into the split's partial (unnormalised output, max, sum) in the workspace.
// A second small kernel merges the splits of each (batch, head).
#include <algorithm>

#include "common.h"

namespace {

constexpr int kDecThreads = 256;
#ifndef DGG_DEC_UNROLL
#define DGG_DEC_UNROLL 8
#endif
constexpr int kUnroll = DGG_DEC_UNROLL;  // key rows per lane group per block (loads in flight per lane: 2 * kUnroll)

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  float* part_o;   // [B, Hq, splits, D]
  float* part_ml;  // [B, Hq, splits, 2]
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_sl;
  int64_t v_sb, v_sh, v_sl;
  int64_t o_sb, o_sh;
  int B, Hq, Hkv, group, L, splits, chunk;
  float c;  // scale * log2(e)
};

// Splits per workgroup: a workgroup runs its splits one after another, writing one partial each, and issues the next
// split's first loads before it merges the current one. Measured at config 5 (64 splits, 2,048 (b, h), identical
// outputs): 1 split per workgroup in this loop 5.18-5.27 ms, 2 splits 5.23-5.27, 4 and 8 5.27-5.31, and the earlier
// for-loop form (loads at the top of each block) 5.27-5.40 ms, in alternating A/Bs on one box. In this loop form the
// compiler issues the next block's loads into a second register set before the current block's exponentials and
// P.V accumulation (194 VGPRs); copying V by hand into a second set for the same effect measured no gain.
constexpr int kSplitsPerWg = 1;
template <typename T, int D>
__global__ void __launch_bounds__(kDecThreads) decode_partial_kernel(DecodeParams p) {
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  constexpr int LPK = D / 8;                 // lanes per key row
  constexpr int GPW = 64 / LPK;              // key rows per wave instruction
  constexpr int GROUPS = GPW * (kDecThreads / 64);  // lane groups per workgroup
  __shared__ float sm[GROUPS], sl[GROUPS];
  __shared__ float so[GROUPS][D + 4];

  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / p.group;
  const int tid = threadIdx.x;
  const int grp = tid / LPK;  // 0..GROUPS-1 (row slot inside one block of key rows)
  const int sub = tid % LPK;  // which 8 head-dim elements
  const int s_end = min(p.splits, (int)(blockIdx.x + 1) * kSplitsPerWg);

  const S* qp = static_cast<const S*>(p.q) + b * p.q_sb + h * p.q_sh;
  const S* kp = static_cast<const S*>(p.k) + b * p.k_sb + hk * p.k_sh + sub * 8;
  const S* vp = static_cast<const S*>(p.v) + b * p.v_sb + hk * p.v_sh + sub * 8;
  f32x8 qv = to_f32x8(ld16<V8>(qp + sub * 8)) * p.c;

  V8 kr[kUnroll], vr[kUnroll];
  bool ok[kUnroll];
  // Loads of the block of GROUPS * kUnroll key rows from `base` of a split ending at k1 > base. Keys past the end
  // re-read its last key (finite; masked to p = 0 below), so that all 2*kUnroll loads go out back to back: a load
  // under a per-lane branch is waited for on its own. Non-temporal: each cache row is read once (5.55 -> 5.33 ms at
  // config 5).
  auto issue = [&](int base, int k1) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int key = base + u * GROUPS + grp;
      ok[u] = key < k1;
      const int kc = min(key, k1 - 1);
      kr[u] = __builtin_nontemporal_load(reinterpret_cast<const V8*>(kp + (int64_t)kc * p.k_sl));
      vr[u] = __builtin_nontemporal_load(reinterpret_cast<const V8*>(vp + (int64_t)kc * p.v_sl));
    }
  };
  int split = blockIdx.x * kSplitsPerWg;
  int k1 = min(p.L, split * p.chunk + p.chunk);
  int base = split * p.chunk;
  if (base < k1) issue(base, k1);
  float m = -INFINITY, l = 0.f;
  f32x8 acc = {};
  while (true) {
    if (base < k1) {
      float s[kUnroll];
      float bm = -INFINITY;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const f32x8 kf = to_f32x8(kr[u]);
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qv[e], kf[e], d);
#pragma unroll
        for (int off = LPK / 2; off >= 1; off >>= 1) d += __shfl_xor(d, off, 64);
        s[u] = ok[u] ? d : -INFINITY;
        bm = fmaxf(bm, s[u]);
      }
      const float m_new = fmaxf(m, bm);
      if (m_new > m) {
        const float alpha = fast_exp2(m - m_new);  // m == -inf -> 0
        l *= alpha;
        acc *= alpha;
        m = m_new;
      }
      const float mu = m == -INFINITY ? 0.f : m;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float pe = fast_exp2(s[u] - mu);
        l += pe;
        acc += pe * to_f32x8(vr[u]);
      }
      base += GROUPS * kUnroll;
      if (base < k1) {
        issue(base, k1);
        continue;
      }
    }
    // The split is done: the next split's first loads go out, then the lane groups' states of this split are merged
    // through LDS into its partial (unnormalised output, max, sum).
    const int nsplit = split + 1;
    const int nbase = nsplit * p.chunk, nk1 = min(p.L, nbase + p.chunk);
    if (nsplit < s_end && nbase < nk1) issue(nbase, nk1);
    if (sub == 0) {
      sm[grp] = m;
      sl[grp] = l;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) so[grp][sub * 8 + e] = acc[e];
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < GROUPS; ++i) M = fmaxf(M, sm[i]);
    const float Mu = M == -INFINITY ? 0.f : M;
    const int64_t pidx = ((int64_t)b * p.Hq + h) * p.splits + split;
    for (int d = tid; d < D; d += kDecThreads) {
      float od = 0.f;
#pragma unroll
      for (int i = 0; i < GROUPS; ++i) od += fast_exp2(sm[i] - Mu) * so[i][d];
      p.part_o[pidx * D + d] = od;
    }
    if (tid == 0) {
      float L = 0.f;
#pragma unroll
      for (int i = 0; i < GROUPS; ++i) L += fast_exp2(sm[i] - Mu) * sl[i];
      p.part_ml[pidx * 2 + 0] = M;
      p.part_ml[pidx * 2 + 1] = L;
    }
    if (nsplit >= s_end) break;
    __syncthreads();  // every lane group has read sm / sl / so before the next split's merge rewrites them
    split = nsplit;
    base = nbase;
    k1 = nk1;
    m = -INFINITY;
    l = 0.f;
    acc = f32x8{};
  }
}

// Merge: o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s, lse = (M + log2 L) ln 2.
template <typename T, int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(DecodeParams p) {
  typedef typename T::scalar S;
  const int h = blockIdx.x, b = blockIdx.y;
  const int64_t base = ((int64_t)b * p.Hq + h) * p.splits;
  __shared__ float red[8];
  float M = -INFINITY;
  for (int s = threadIdx.x; s < p.splits; s += blockDim.x) M = fmaxf(M, p.part_ml[(base + s) * 2]);
  M = wave_max(M);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = M;
  __syncthreads();
  M = -INFINITY;
  for (int i = 0; i < (int)(blockDim.x + 63) / 64; ++i) M = fmaxf(M, red[i]);
  const float Mu = M == -INFINITY ? 0.f : M;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float od = 0.f, L = 0.f;
    for (int s = 0; s < p.splits; ++s) {
      const float wgt = fast_exp2(p.part_ml[(base + s) * 2] - Mu);
      L += wgt * p.part_ml[(base + s) * 2 + 1];
      od += wgt * p.part_o[(base + s) * D + d];
    }
    static_cast<S*>(p.o)[b * p.o_sb + h * p.o_sh + d] = to_s<S>(od / L);
    if (d == 0 && p.lse != nullptr) p.lse[(int64_t)b * p.Hq + h] = (M == -INFINITY ? -INFINITY : M + fast_log2(L)) * kLn2;
  }
}

template <typename T, int D>
void launch_decode(const DecodeParams& p, hipStream_t st) {
  hipLaunchKernelGGL((decode_partial_kernel<T, D>), dim3((p.splits + kSplitsPerWg - 1) / kSplitsPerWg, p.Hq, p.B), dim3(kDecThreads), 0, st, p);
  hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3(p.Hq, p.B), dim3(D < 256 ? 128 : 256), 0, st, p);
}

}  // namespace

extern "C" int64_t dgg_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t D, int64_t splits) {
  if (B < 0 || Hq < 0 || D < 0 || splits < 0) return -1;
  return B * Hq * splits * (D + 2) * (int64_t)sizeof(float);
}

namespace dgg {

// Shared body of dgg_attn_decode and dgg_attn_decode_noalloc (declared in common.h).
int decode_launch(const char* op, const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                  int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                  const int64_t* strides, int64_t splits, float scale, int dtype, void* stream,
                  int (*resolve_ws)(const char* op, void* stream, void** ws)) {
  const bool use_scratch = resolve_ws != nullptr;
  DGG_REQUIRE(dtype == DGG_F16 || dtype == DGG_BF16, DGG_ERR_DTYPE,
              "%s: dtype code %d not supported (attention kernels take f16 or bf16)", op, dtype);
  DGG_REQUIRE(D == 64 || D == 128 || D == 256, DGG_ERR_UNSUPPORTED, "%s: head_dim %lld not supported (64, 128, 256)",
              op, (long long)D);
  DGG_REQUIRE(B >= 0 && B < 65536 && Hq > 0 && Hq < 65536 && Hkv > 0 && Hq % Hkv == 0, DGG_ERR_SHAPE,
              "%s: bad batch/head sizes (B=%lld Hq=%lld Hkv=%lld)", op, (long long)B, (long long)Hq, (long long)Hkv);
  DGG_REQUIRE(L >= 1 && L < (1ll << 31), DGG_ERR_SHAPE, "%s: kv length must be in [1, 2^31) (got %lld)", op,
              (long long)L);
  DGG_REQUIRE(splits >= 1 && splits <= 1024, DGG_ERR_SHAPE, "%s: splits must be in [1, 1024] (got %lld)", op,
              (long long)splits);
  DGG_REQUIRE(std::isfinite(scale) && scale > 0.f, DGG_ERR_SHAPE, "%s: scale must be finite and > 0", op);
  DGG_REQUIRE(strides != nullptr, DGG_ERR_NULL, "%s: strides is NULL", op);
  for (int i = 0; i < 10; ++i)
    DGG_REQUIRE(strides[i] >= 0 && strides[i] % 8 == 0, DGG_ERR_STRIDE,
                "%s: stride[%d] = %lld must be a non-negative multiple of 8 elements", op, i, (long long)strides[i]);
  const int64_t need = dgg_attn_decode_workspace_bytes(B, Hq, D, splits);
  if (use_scratch)
    DGG_REQUIRE(need <= workspace_bytes, DGG_ERR_WORKSPACE,
                "%s: the split partials need %lld bytes, more than the fixed scratch of %lld bytes (use fewer splits, "
                "or dgg_attn_decode with a workspace)", op, (long long)need, (long long)workspace_bytes);
  else
    DGG_REQUIRE(workspace_bytes >= need, DGG_ERR_WORKSPACE, "%s: workspace of %lld bytes < required %lld", op,
                (long long)workspace_bytes, (long long)need);
  if (B == 0) return DGG_OK;
  DGG_REQUIRE(q && k && v && o, DGG_ERR_NULL, "%s: null pointer", op);
  if (Hq > Hkv) {
    // Grouped query heads: the split-KV kernels take the G query heads of a KV head as the rows of one workgroup, so
    // each cache row is read once, not once per query head. The cache [B, Hkv, L, D] is their [B, Sk, Hkv, D] with
    // strides {b, l, h}; the partials have the same size.
    const int64_t st12[12] = {strides[0], 0,          strides[1], strides[2], strides[4], strides[3],
                              strides[5], strides[7], strides[6], strides[8], 0,          strides[9]};
    return dgg::splitkv_launch(op, q, k, v, o, lse, workspace, workspace_bytes, B, 1, L, Hq, Hkv, D, st12, splits,
                               scale, 0.f, 0, 0u, dtype, stream, resolve_ws);
  }
  if (use_scratch) {
    if (int rc = resolve_ws(op, stream, &workspace)) return rc;
  }
  DGG_REQUIRE(workspace != nullptr, DGG_ERR_NULL, "%s: null workspace", op);
  DGG_REQUIRE(dgg::aligned16(q) && dgg::aligned16(k) && dgg::aligned16(v) && dgg::aligned16(workspace),
              DGG_ERR_ALIGN, "%s: q/k/v/workspace must be 16-byte aligned", op);
  DecodeParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.lse = lse;
  p.part_o = static_cast<float*>(workspace);
  p.part_ml = p.part_o + B * Hq * splits * D;
  p.q_sb = strides[0]; p.q_sh = strides[1];
  p.k_sb = strides[2]; p.k_sh = strides[3]; p.k_sl = strides[4];
  p.v_sb = strides[5]; p.v_sh = strides[6]; p.v_sl = strides[7];
  p.o_sb = strides[8]; p.o_sh = strides[9];
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.group = (int)(Hq / Hkv);
  p.L = (int)L;
  p.splits = (int)splits;
  p.chunk = (int)((L + splits - 1) / splits);
  p.c = scale * kLog2e;
  hipStream_t st = dgg::as_stream(stream);
  if (dtype == DGG_BF16) {
    if (D == 64) launch_decode<BF16, 64>(p, st);
    else if (D == 128) launch_decode<BF16, 128>(p, st);
    else launch_decode<BF16, 256>(p, st);
  } else {
    if (D == 64) launch_decode<F16, 64>(p, st);
    else if (D == 128) launch_decode<F16, 128>(p, st);
    else launch_decode<F16, 256>(p, st);
  }
  return dgg::check_launch(op);
}

}  // namespace dgg

extern "C" int dgg_attn_decode(const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                               int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                               const int64_t* strides, int64_t splits, float scale, int dtype, void* stream) {
  return dgg::decode_launch("attn_decode", q, k, v, o, lse, workspace, workspace_bytes, B, Hq, Hkv, L, D, strides,
                            splits, scale, dtype, stream, nullptr);
}
