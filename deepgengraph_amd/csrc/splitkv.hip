// Split-KV attention for a few query rows over a long key range: multi-row decode, chunked prefill and speculative
// verification (Attn.forward with 1 < q_len << kv_len, attn.py:18-34, under the bottom-right causal mask of
// attn.py:22-23), and grouped-query decode (q_len 1, several query heads per KV head, the convention of
// roco.py:25-27).
//
// Rows. The query rows of one (batch, KV head) are its G = Hq / Hkv query heads times the Sq query rows, row
// r = qh * Sq + i (query head hk * G + qh, query row i). A workgroup takes 32 * NW of them, one wave per 32 rows,
// and one slice ("split") of the keys, so every K / V row of a KV head crosses HBM once per 32 * NW query rows, not
// once per query head and row. Each split writes an unnormalised partial (O, row maximum, row sum) per row; a merge
// kernel combines the splits of each row as the decode merge does.
//
// Tile loop. Keys in tiles of 32: the workgroup copies K and V rows global -> registers (16-byte loads, consecutive
// lanes on consecutive chunks of a row) -> LDS (rows padded by 16 bytes), one tile ahead of the compute. Each wave then runs
//   S^T (32 keys x 32 rows) = K . Q^T     v_mfma_f32_32x32x16, A = K fragments from LDS, B = Q in registers
//   O^T (D x 32 rows)      += V^T . P^T   A = V^T by transposing LDS reads, B = P straight from the S^T accumulator
// with the online softmax of the prefill kernels (one query row per lane, the cross-half exchange, lazy rescale).
// Tiles every row of a wave sees in full skip the per-element mask; tiles no row of the wave sees are skipped.
// The MFMA work per byte is small (a few rows per key): the loop is bound by the K / V stream.
#include <climits>

#include "common.h"

#include "attention_common.h"

namespace dgg_attn {
namespace {

constexpr int kSkBN = 32;  // keys per tile

struct SplitParams {
  AttnParams a;     // pointers, strides, sizes, mask and soft-cap constants
  float* part_o;    // [B, Hkv, M, splits, D] unnormalised partial outputs
  float* part_ml;   // [B, Hkv, M, splits, 2] (row maximum in the exp2 domain, row sum)
  int M;            // rows per KV head: G * Sq
  int n_rg;         // row groups (of 32 * NW rows) per KV head
  int splits;
  int chunk;        // keys per split (a multiple of kSkBN)
  int k_first;      // first key any row sees (sliding window); splits cover [k_first, Sk)
};

__device__ __forceinline__ int wave_imin(int x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = min(x, __shfl_xor(x, off, 64));
  return x;
}
__device__ __forceinline__ int wave_imax(int x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = max(x, __shfl_xor(x, off, 64));
  return x;
}

// Registers: at head_dim 64 and 128 two waves per SIMD (231 VGPRs at 128, no spills), so that the K / V stream has
// enough loads in flight; head_dim 256 (Q 64 + O 128 registers) runs one wave per SIMD with two waves per workgroup.
template <typename T, int D, int NW, bool SOFTCAP>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(D >= 256 ? 1 : 2)))
attn_splitkv_kernel(SplitParams sp) {
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  typedef typename T::vec4 V4;
  const AttnParams& p = sp.a;
  constexpr int BN = kSkBN;
  constexpr int KP = D + 8;             // padded row (elements): 16-byte shift per row for both read patterns
  constexpr int NKK = D / 16;           // MFMA k-steps over the head dim
  constexpr int NDB = D / 32;           // 32-wide head-dim blocks of O^T
  constexpr int NPK = BN / 16;          // MFMA k-steps over the keys of a tile in P.V
  constexpr int NT = 64 * NW;
  constexpr int LPR = D / 8;            // threads per key row: consecutive lanes read consecutive 16-byte chunks
  constexpr int RPI = NT / LPR;         // key rows per load instruction of the workgroup
  constexpr int CPT = BN / RPI;         // 16-byte chunks per thread per tile (K and V each)
  static_assert(CPT * RPI == BN && RPI * LPR == NT, "tile mapping");

  __shared__ __attribute__((aligned(16))) S Ks[BN][KP];
  __shared__ __attribute__((aligned(16))) S Vs[BN][KP];

  const int split = blockIdx.x;
  const int hk = blockIdx.y / sp.n_rg, rg = blockIdx.y - hk * sp.n_rg;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r = lane & 31, g = lane >> 5;
  const int tr_krow = (lane & 15) >> 2;                           // key row within a group of 4
  const int tr_dcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);  // head-dim column within a 32-wide block

  // This lane's row (query column of S^T): lanes r and r + 32 share it.
  const int row = (rg * NW + w) * 32 + r;
  const bool row_ok = row < sp.M;
  const int rowc = row_ok ? row : sp.M - 1;
  const int qh = rowc / p.Sq, qi = rowc - qh * p.Sq;
  const int h = hk * p.group + qh;

  // Q fragment (B operand of S^T = K.Q^T): query row qi of head h, head-dim elements 16kk + 8g .. +8.
  const S* qp = static_cast<const S*>(p.q) + b * p.q_sb + (int64_t)qi * p.q_ss + (int64_t)h * p.q_sh;
  V8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) qf[kk] = ld16<V8>(qp + 16 * kk + 8 * g);
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    asm volatile("" : "+v"(qf[kk]));
    if (!row_ok) qf[kk] = V8{};
  }

  // Keys of this split, and the keys this lane's row sees in it: k_lo <= key <= k_hi.
  const int k0 = sp.k_first + split * sp.chunk;
  const int k1 = min(p.Sk, k0 + sp.chunk);
  int k_hi = k1 - 1, k_lo = k0;
  if (p.causal) k_hi = min(k_hi, qi + p.offset);
  if (p.window > 0) k_lo = max(k_lo, qi + p.offset - p.window + 1);
  if (!row_ok) k_hi = k_lo - 1;
  // Wave-uniform tile classes: a tile inside [lo_max, hi_min] is seen whole by every row of the wave (a row with no
  // key in the split makes every tile masked; lanes past the last row, whose results are dropped, do not count); a
  // tile outside [lo_min, hi_max] is seen by none.
  const bool empty = k_hi < k_lo;
  const int lo_max = wave_imax(!row_ok ? INT_MIN : empty ? INT_MAX : k_lo);
  const int hi_min = wave_imin(!row_ok ? INT_MAX : empty ? INT_MIN : k_hi);
  const int lo_min = wave_imin(row_ok && !empty ? k_lo : INT_MAX);
  const int hi_max = wave_imax(row_ok && !empty ? k_hi : INT_MIN);

  const int n_t = k1 > k0 ? (k1 - k0 + BN - 1) / BN : 0;
  // Load i of a tile: thread tid reads 16-byte chunk tid % LPR of tile row i * RPI + tid / LPR, so one wave
  // instruction covers 64 / LPR whole rows.
  const int row0 = tid / LPR, c0 = tid % LPR;
  const S* kp = static_cast<const S*>(p.k) + b * p.k_sb + (int64_t)hk * p.k_sh + c0 * 8;
  const S* vp = static_cast<const S*>(p.v) + b * p.v_sb + (int64_t)hk * p.v_sh + c0 * 8;
  V8 kreg[CPT], vreg[CPT];
  // Rows past the split's end re-read its last key (masked below, finite: contributes exactly 0). Each K / V row is
  // read once, so the loads are non-temporal: measured at q_len 4 over 32K keys, 90.3-90.6 against 101.3-101.5 us
  // with ordinary loads (the stream alone, without the tile compute, runs the same times: the loop is bound by it).
  auto load = [&](int t) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int key = min(k0 + t * BN + i * RPI + row0, k1 - 1);
      kreg[i] = __builtin_nontemporal_load(reinterpret_cast<const V8*>(kp + (int64_t)key * p.k_ss));
      vreg[i] = __builtin_nontemporal_load(reinterpret_cast<const V8*>(vp + (int64_t)key * p.v_ss));
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      *reinterpret_cast<V8*>(&Ks[i * RPI + row0][c0 * 8]) = kreg[i];
      *reinterpret_cast<V8*>(&Vs[i * RPI + row0][c0 * 8]) = vreg[i];
    }
  };

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) oacc[i] = f32x16{};
  float m_run = -INFINITY;  // reference maximum (value units)
  float l_part[4] = {0.f, 0.f, 0.f, 0.f};
  const float c = score_coeff<SOFTCAP, 0>(p);

  auto tile = [&](const int kt, auto masked) {
    f32x16 sacc = f32x16{};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const V8 a = *reinterpret_cast<const V8*>(&Ks[r][16 * kk + 8 * g]);
      sacc = mfma32(a, qf[kk], sacc);
    }
    // element j holds key kt + 8*(j/4) + 4g + j%4
    const int rel_hi = k_hi - (kt + 4 * g), rel_lo = k_lo - (kt + 4 * g);
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float x = score_value<T, SOFTCAP, 0>(sacc[j], p);
      if constexpr (decltype(masked)::value) {
        const int o = 8 * (j >> 2) + (j & 3);
        x = (o <= rel_hi && o >= rel_lo) ? x : -INFINITY;
      }
      sacc[j] = x;
      mloc = fmaxf(mloc, x);
    }
    mloc = half_swap_max(mloc);
    const float m_new = fmaxf(m_run, mloc);
    const bool need = m_new * c > m_run * c + kRescaleThreshold;
    if (__any(need)) {
      const float alpha = need ? fast_exp2((m_run - m_new) * c) : 1.0f;
      if (need) m_run = m_new;
#pragma unroll
      for (int i = 0; i < 4; ++i) l_part[i] *= alpha;
#pragma unroll
      for (int i = 0; i < NDB; ++i) oacc[i] *= alpha;
    }
    const float mc = m_run == -INFINITY ? 0.f : m_run * c;
#pragma unroll
    for (int kk = 0; kk < NPK; ++kk) {
      f32x8 pv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = fast_exp2(fmaf(sacc[8 * kk + e], c, -mc));
        l_part[e & 3] += pe;
        pv[e] = pe;
      }
      const V8 pb = from_f32x8<V8>(pv);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        // A = V^T rows db*32 + r, keys 16kk + 4g + {0..3} and 16kk + 8 + 4g + {0..3} (the P operand's key order)
        const S* vrow = &Vs[16 * kk + 4 * g + tr_krow][db * 32 + tr_dcol];
        const V4 lo = tr_read(vrow);
        const V4 hi = tr_read(vrow + 8 * KP);
        oacc[db] = mfma32(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), pb, oacc[db]);
      }
    }
  };

  if (n_t > 0) load(0);
  for (int t = 0; t < n_t; ++t) {
    store();
    __syncthreads();
    if (t + 1 < n_t) load(t + 1);  // in flight during this tile's compute
    const int kt = k0 + t * BN;
    if (kt <= hi_max && kt + BN - 1 >= lo_min) {
      if (kt >= lo_max && kt + BN - 1 <= hi_min) tile(kt, std::false_type{});
      else tile(kt, std::true_type{});
    }
    __syncthreads();
  }

  // Partial of this split for the lane's row: unnormalised O, maximum (exp2 domain), sum.
  const float l_run = (l_part[0] + l_part[1]) + (l_part[2] + l_part[3]);
  const float l_tot = half_swap_sum(l_run);
  if (row_ok) {
    const int64_t pidx = (((int64_t)b * p.Hkv + hk) * sp.M + row) * sp.splits + split;
    float* po = sp.part_o + pidx * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const f32x4 ov = {oacc[db][4 * jj], oacc[db][4 * jj + 1], oacc[db][4 * jj + 2], oacc[db][4 * jj + 3]};
        *reinterpret_cast<f32x4*>(po + db * 32 + 8 * jj + 4 * g) = ov;
      }
    }
    if (g == 0) {
      sp.part_ml[pidx * 2 + 0] = m_run == -INFINITY ? -INFINITY : m_run * c;
      sp.part_ml[pidx * 2 + 1] = l_tot;
    }
  }
}

// Merge of the splits of one row: o = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, lse = M + log2 L (base 2, or
// times ln 2). A row that sees no key at all gets L = 0, so o = NaN (the reference's softmax of an all -inf row)
// and lse = -inf. 256 threads per row: the weights go to LDS, then each thread sums 4 head-dim columns over every
// (256 / (D/4))-th split (16-byte loads, four splits in flight) and the groups are added through LDS.
constexpr int kMergeThreads = 256;
template <typename T, int D>
__global__ void __launch_bounds__(kMergeThreads) attn_splitkv_merge_kernel(SplitParams sp) {
  typedef typename T::scalar S;
  const AttnParams& p = sp.a;
  constexpr int kMaxSplits = 1024;
  constexpr int CPR = D / 4;                    // float4 columns per row
  constexpr int NG = kMergeThreads / CPR;       // split groups
  __shared__ float wts[kMaxSplits];
  __shared__ f32x4 part[NG][CPR];
  __shared__ float red[kMergeThreads / 64][2];
  const int row = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wv = tid >> 6;
  const int64_t base = (((int64_t)b * p.Hkv + hk) * sp.M + row) * sp.splits;
  const float* ml = sp.part_ml + base * 2;
  float M = -INFINITY;
  for (int s = tid; s < sp.splits; s += kMergeThreads) M = fmaxf(M, ml[2 * s]);
  M = wave_max(M);
  if ((tid & 63) == 0) red[wv][0] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0][0], red[1][0]), fmaxf(red[2][0], red[3][0]));
  const float Mu = M == -INFINITY ? 0.f : M;
  float L = 0.f;
  for (int s = tid; s < sp.splits; s += kMergeThreads) {
    const float wgt = fast_exp2(ml[2 * s] - Mu);
    wts[s] = wgt;
    L += wgt * ml[2 * s + 1];
  }
  L = wave_sum(L);
  if ((tid & 63) == 0) red[wv][1] = L;
  __syncthreads();
  L = (red[0][1] + red[1][1]) + (red[2][1] + red[3][1]);
  const int col = tid % CPR, grp = tid / CPR;
  const float* po = sp.part_o + base * D + 4 * col;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int s = grp;
  for (; s + 3 * NG < sp.splits; s += 4 * NG) {
    const f32x4 a0 = *reinterpret_cast<const f32x4*>(po + (int64_t)s * D);
    const f32x4 a1 = *reinterpret_cast<const f32x4*>(po + (int64_t)(s + NG) * D);
    const f32x4 a2 = *reinterpret_cast<const f32x4*>(po + (int64_t)(s + 2 * NG) * D);
    const f32x4 a3 = *reinterpret_cast<const f32x4*>(po + (int64_t)(s + 3 * NG) * D);
    acc += wts[s] * a0 + wts[s + NG] * a1 + wts[s + 2 * NG] * a2 + wts[s + 3 * NG] * a3;
  }
  for (; s < sp.splits; s += NG) acc += wts[s] * *reinterpret_cast<const f32x4*>(po + (int64_t)s * D);
  part[grp][col] = acc;
  __syncthreads();
  const int qh = row / p.Sq, qi = row - qh * p.Sq;
  const int h = hk * p.group + qh;
  if (tid < CPR) {
    f32x4 o = part[0][tid];
#pragma unroll
    for (int gi = 1; gi < NG; ++gi) o += part[gi][tid];
    const float inv = 1.0f / L;
    S* op = static_cast<S*>(p.o) + b * p.o_sb + (int64_t)qi * p.o_ss + (int64_t)h * p.o_sh + 4 * tid;
#pragma unroll
    for (int e = 0; e < 4; ++e) op[e] = to_s<S>(o[e] * inv);
  }
  if (tid == 0 && p.lse != nullptr) {
    const float l2 = M == -INFINITY ? -INFINITY : M + fast_log2(L);
    p.lse[((int64_t)b * p.Hq + h) * p.Sq + qi] = p.lse_base2 ? l2 : l2 * kLn2;
  }
}

template <typename T, int D, int NW>
void launch_splitkv(const SplitParams& sp, hipStream_t st) {
  const dim3 grid(sp.splits, sp.a.Hkv * sp.n_rg, sp.a.B);
  if (sp.a.softcap > 0.f)
    hipLaunchKernelGGL((attn_splitkv_kernel<T, D, NW, true>), grid, dim3(64 * NW), 0, st, sp);
  else
    hipLaunchKernelGGL((attn_splitkv_kernel<T, D, NW, false>), grid, dim3(64 * NW), 0, st, sp);
  hipLaunchKernelGGL((attn_splitkv_merge_kernel<T, D>), dim3(sp.M, sp.a.Hkv, sp.a.B), dim3(kMergeThreads), 0, st,
                     sp);
}

template <typename T, int D>
void pick_splitkv(const SplitParams& sp, int nw, hipStream_t st) {
  if constexpr (D >= 256) launch_splitkv<T, D, 2>(sp, st);
  else if (nw == 1) launch_splitkv<T, D, 1>(sp, st);
  else launch_splitkv<T, D, 2>(sp, st);
}

}  // namespace
}  // namespace dgg_attn

namespace dgg {

// Shared body of dgg_attn_splitkv and of dgg_attn_decode / dgg_attn_decode_noalloc for grouped query heads (declared
// in common.h).
int splitkv_launch(const char* op, const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                   int64_t workspace_bytes, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D,
                   const int64_t* strides, int64_t splits, float scale, float softcap, int64_t window, uint32_t flags,
                   int dtype, void* stream, int (*resolve_ws)(const char* op, void* stream, void** ws)) {
  using namespace dgg_attn;
  if (int rc = validate_attn(op, q, k, B, Sq, Sk, Hq, Hkv, D, strides, 12, scale, softcap, window, dtype)) return rc;
  DGG_REQUIRE(dtype == DGG_F16 || dtype == DGG_BF16, DGG_ERR_DTYPE, "%s: split-KV takes f16 or bf16 (dtype code %d)",
              op, dtype);
  DGG_REQUIRE((flags & DGG_ATTN_REF_ROUNDING) == 0, DGG_ERR_UNSUPPORTED,
              "%s: reference rounding is not supported by the split-KV kernels (use dgg_attn_prefill)", op);
  DGG_REQUIRE(Sq >= 1 && Sk >= 1, DGG_ERR_SHAPE, "%s: Sq and Sk must be >= 1 (got %lld, %lld)", op, (long long)Sq,
              (long long)Sk);
  DGG_REQUIRE(splits >= 1 && splits <= 1024, DGG_ERR_SHAPE, "%s: splits must be in [1, 1024] (got %lld)", op,
              (long long)splits);
  const int64_t M = (Hq / Hkv) * Sq;
  DGG_REQUIRE(M < 65536 && Hkv * ((M + 63) / 64) < 65536 && B < 65536, DGG_ERR_SHAPE,
              "%s: too many rows per KV head (%lld), KV heads or batch entries for the grid", op, (long long)M);
  const int64_t need = dgg_attn_splitkv_workspace_bytes(B, Sq, Hq, D, splits);
  DGG_REQUIRE(workspace_bytes >= need, DGG_ERR_WORKSPACE, "%s: the split partials need %lld bytes, workspace is %lld",
              op, (long long)need, (long long)workspace_bytes);
  if (B == 0) return DGG_OK;
  DGG_REQUIRE(o && v, DGG_ERR_NULL, "%s: null v/o pointer", op);
  DGG_REQUIRE(dgg::aligned16(v) && dgg::aligned16(o), DGG_ERR_ALIGN, "%s: v/o must be 16-byte aligned", op);
  if (resolve_ws != nullptr) {
    if (int rc = resolve_ws(op, stream, &workspace)) return rc;
  }
  DGG_REQUIRE(workspace != nullptr, DGG_ERR_NULL, "%s: null workspace", op);
  DGG_REQUIRE(dgg::aligned16(workspace), DGG_ERR_ALIGN, "%s: workspace must be 16-byte aligned", op);

  SplitParams sp{};
  sp.a = make_params(q, k, v, o, B, Sq, Sk, Hq, Hkv, D, scale, softcap, window, flags);
  AttnParams& p = sp.a;
  p.lse = lse;
  p.q_sb = strides[0]; p.q_ss = strides[1]; p.q_sh = strides[2];
  p.k_sb = strides[3]; p.k_ss = strides[4]; p.k_sh = strides[5];
  p.v_sb = strides[6]; p.v_ss = strides[7]; p.v_sh = strides[8];
  p.o_sb = strides[9]; p.o_ss = strides[10]; p.o_sh = strides[11];
  sp.M = (int)M;
  // one wave per 32 rows, two for more rows (and always two at head_dim 256, whose single wave would spill)
  const int nw = M <= 32 && D < 256 ? 1 : 2;
  sp.n_rg = (int)((M + 32 * nw - 1) / (32 * nw));
  // Keys any row sees: [k_first, Sk). Row 0 has the lowest window edge; under the causal mask the last row sees
  // key Sk - 1.
  const int64_t k_first = window > 0 ? std::max<int64_t>(0, (Sk - Sq) - window + 1) : 0;
  const int64_t span = Sk - k_first;
  int64_t chunk = (span + splits - 1) / splits;
  chunk = (chunk + kSkBN - 1) / kSkBN * kSkBN;
  sp.k_first = (int)k_first;
  sp.chunk = (int)chunk;
  sp.splits = (int)splits;
  sp.part_o = static_cast<float*>(workspace);
  sp.part_ml = sp.part_o + B * Hq * Sq * splits * D;
  hipStream_t st = dgg::as_stream(stream);
  if (dtype == DGG_BF16) {
    if (D == 64) pick_splitkv<BF16, 64>(sp, nw, st);
    else if (D == 128) pick_splitkv<BF16, 128>(sp, nw, st);
    else pick_splitkv<BF16, 256>(sp, nw, st);
  } else {
    if (D == 64) pick_splitkv<F16, 64>(sp, nw, st);
    else if (D == 128) pick_splitkv<F16, 128>(sp, nw, st);
    else pick_splitkv<F16, 256>(sp, nw, st);
  }
  return dgg::check_launch(op);
}

}  // namespace dgg

extern "C" int64_t dgg_attn_splitkv_workspace_bytes(int64_t B, int64_t Sq, int64_t Hq, int64_t D, int64_t splits) {
  if (B < 0 || Sq < 0 || Hq < 0 || D < 0 || splits < 0) return -1;
  return B * Hq * Sq * splits * (D + 2) * (int64_t)sizeof(float);
}

extern "C" int dgg_attn_splitkv(const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                                int64_t workspace_bytes, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv,
                                int64_t D, const int64_t* strides, int64_t splits, float scale, float softcap,
                                int64_t window, uint32_t flags, int dtype, void* stream) {
  return dgg::splitkv_launch("attn_splitkv", q, k, v, o, lse, workspace, workspace_bytes, B, Sq, Sk, Hq, Hkv, D,
                             strides, splits, scale, softcap, window, flags, dtype, stream, nullptr);
}
