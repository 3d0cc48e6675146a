// Fused online-softmax attention for gfx950 (CDNA4): prefill forward (causal / sliding window / tanh soft-cap /
// GQA), the column-score passes of the selection cases (H2O, RoCo, SnapKV, Corm, KeyFormer) and KeyFormer's
// perturbed row log-sum-exp.
//
// Products. Both run on v_mfma_f32_32x32x16_{bf16,f16} with the scores computed transposed:
//   S^T (BN x 32)  = K (BN x D) . Q^T (D x 32)     A = K fragments from LDS, B = Q held in registers
//   O^T (D x 32)  += V^T (D x BN) . P^T (BN x 32)  A = V^T by transposing LDS reads (ds_read_b64_tr_b16) of the
//                                                   row-major V tile, B = P straight from the S^T accumulator
// One query per lane (column n = lane % 32): the row max and row sum are in-lane plus one cross-half exchange
// (v_permlane32_swap), and the accumulator, rounded to 16 bits, is already the B operand of P.V.
// Softmax runs in the exp2 domain with a lazily-updated row maximum: O and l are rescaled only when a row's
// maximum grows by more than 2^8.
//
// Kernels. attn_fwd_dma_kernel (head_dim 128: 8 waves x 32 rows, 128-key tiles; head_dim 256: 4 waves, 64-key
// tiles) copies K/V tiles global -> LDS with direct loads (global_load_lds_dwordx4) into a swizzled ring;
// attn_fwd_kernel (head_dim 64) stages them through registers. Tiles a wave cannot see are skipped, and within
// masked tiles dead 32-key blocks skip their MFMAs. attn_colsum_d128_kernel / attn_colsum_kernel recompute
// P = exp2(s - lse) with one key per lane and sum (or test) it over the queries; attn_kf_rowlse_kernel is the
// row pass of KeyFormer's perturbed softmax. Reference rounding (DGG_ATTN_REF_ROUNDING) rounds the scores as
// the reference does on the GPU: matmul result to the input dtype, then the fp32 multiply by the reciprocal of
// sqrt(D) (and of the soft-cap), rounded again.
// Workgroups are ordered longest-first and grouped by head inside each XCD so the K/V of a head stay in one L2.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.h"

#include "attention_common.h"

// DGG_SPREAD_COPIES (default 1): mask-free tiles of the direct-load forward issue the next tile's copies among their
// QK^T MFMAs; 0 issues them all right after the barrier (for A/B measurements).
#ifndef DGG_SPREAD_COPIES
#define DGG_SPREAD_COPIES 1
#endif

namespace {

using namespace dgg_attn;

// ------------------------------------------------------------------------------------------------
// Forward kernel.
// ------------------------------------------------------------------------------------------------
template <typename T, int D, int BN, bool MASK, bool SOFTCAP, int REFROUND>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(D >= 256 ? 1 : 2, 2))) attn_fwd_kernel(AttnParams p) {
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  typedef typename T::vec4 V4;
  constexpr int KP = D + 8;  // padded K row (elements): 16-byte shift per row for the fragment reads
  constexpr int VP = D + 8;  // padded V row (elements): 16-byte shift per row for the transposing reads
  constexpr int NKK = D / 16;      // MFMA k-steps over the head dim
  constexpr int NMB = BN / 32;     // 32-key blocks per tile
  constexpr int NDB = D / 32;      // 32-wide head-dim blocks of O^T
  constexpr int NPK = BN / 16;     // MFMA k-steps over keys in P.V
  constexpr int CHUNKS = BN * D / 8;
  constexpr int CPT = CHUNKS / kThreads;  // 16-byte chunks per thread per tile (K and V each)
  static_assert(CHUNKS % kThreads == 0, "tile must split evenly over the workgroup");

  __shared__ __attribute__((aligned(16))) S Ks[2][BN][KP];
  __shared__ __attribute__((aligned(16))) S Vs[2][BN][VP];

  int qt, bh;
  map_block(p.n_tiles, p.B * p.Hq, true, qt, bh);
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / p.group;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r = lane & 31, g = lane >> 5;
  const int q0 = qt * kBM;
  const int qi = q0 + 32 * w + r;  // this lane's query row
  const int tr_krow = (lane & 15) >> 2;                              // key row within a group of 4
  const int tr_dcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);     // head-dim column within a 32-wide block

  const S* qp = static_cast<const S*>(p.q) + b * p.q_sb + h * p.q_sh;
  const S* kp = static_cast<const S*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const S* vp = static_cast<const S*>(p.v) + b * p.v_sb + hk * p.v_sh;

  // Q fragment (B operand of S^T = K.Q^T): lane holds query qi, head-dim elements 16kk + 8g .. +8.
  V8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)  // back-to-back loads (rows past the end read the last row, zeroed below)
    qf[kk] = ld16<V8>(qp + (int64_t)min(qi, p.Sq - 1) * p.q_ss + 16 * kk + 8 * g);
  // Re-define the Q registers here (after their loads complete) so that the main loop's wait counting does not
  // treat them as results of outstanding vector-memory loads.
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    asm volatile("" : "+v"(qf[kk]));
    if (qi >= p.Sq) qf[kk] = V8{};
  }

  // Key range of this query tile.
  const int q_last = min(q0 + kBM, p.Sq) - 1;
  int k_begin = 0, k_end = p.Sk;
  if (p.causal) k_end = min(p.Sk, q_last + p.offset + 1);
  if (p.window > 0) k_begin = max(0, q0 + p.offset - p.window + 1);
  const int t_begin = k_begin / BN;
  const int t_end = k_end > k_begin ? (k_end + BN - 1) / BN : t_begin;

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) oacc[i] = f32x16{};
  float m_run = -INFINITY;  // reference maximum (value units)
  const float c = score_coeff<SOFTCAP, REFROUND>(p);

  // Global -> register staging of one K/V tile: each thread owns CPT adjacent 16-byte chunks of one key row of
  // K and of V (coalesced rows; both stay row-major in LDS). Full tiles are addressed through two per-lane
  // pointers that advance by one tile right before each load (so a pointer register is never rewritten while
  // loads through it are in flight), the chunk index going into the immediate offset.
  V8 kreg[CPT], vreg[CPT];
  constexpr int TPR = (D / 8) / CPT;        // threads per row
  static_assert(TPR * CPT == D / 8 && kThreads / TPR == BN, "tile mapping");
  const int k_row0 = tid / TPR, k_c0 = (tid % TPR) * CPT;
  const int64_t k_step = (int64_t)BN * p.k_ss * (int64_t)sizeof(S), v_step = (int64_t)BN * p.v_ss * (int64_t)sizeof(S);
  // pointers of tile t_begin - 1 (advanced before use)
  gptr k_addr = to_gptr(kp + (int64_t)(k_row0 - BN) * p.k_ss + k_c0 * 8) + (int64_t)t_begin * k_step;
  gptr v_addr = to_gptr(vp + (int64_t)(k_row0 - BN) * p.v_ss + k_c0 * 8) + (int64_t)t_begin * v_step;
  auto load_full = [&]() {
    k_addr += k_step;
    v_addr += v_step;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      kreg[i] = ldg16<V8>(k_addr + 16 * i);
      vreg[i] = ldg16<V8>(v_addr + 16 * i);
    }
  };
  // Ragged last tile: rows past the end are clamped to the last row (masked, finite: contributes exactly 0).
  auto load_ragged = [&](int t) {
    k_addr += k_step;
    v_addr += v_step;
    const int kb = t * BN;
    const int kr = min(k_row0, p.Sk - 1 - kb);  // >= 0 for every loaded tile
    const S* kt = kp + (int64_t)(kb + kr) * p.k_ss + k_c0 * 8;
    const S* vt = vp + (int64_t)(kb + kr) * p.v_ss + k_c0 * 8;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      kreg[i] = ld16<V8>(kt + i * 8);
      vreg[i] = ld16<V8>(vt + i * 8);
    }
  };
  auto tile_full = [&](int t) { return (t + 1) * BN <= p.Sk; };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      *reinterpret_cast<V8*>(&Ks[buf][k_row0][(k_c0 + i) * 8]) = kreg[i];
      *reinterpret_cast<V8*>(&Vs[buf][k_row0][(k_c0 + i) * 8]) = vreg[i];
    }
  };

  if (t_begin < t_end) {
    if (tile_full(t_begin)) load_full();
    else load_ragged(t_begin);
    store_tile(0);
  }
  __syncthreads();

  // Visible keys of this lane's query: lo <= key <= hi (bottom-right causal, sliding window, ragged end).
  int k_hi = p.Sk - 1, k_lo = 0;
  if (p.causal) k_hi = min(k_hi, qi + p.offset);
  if (p.window > 0) k_lo = max(k_lo, qi + p.offset - p.window + 1);
  float l_part[4] = {0.f, 0.f, 0.f, 0.f};  // split row sums (breaks the dependent add chain)

  // One K/V tile: S^T = K.Q^T, scores, online softmax, O^T += V^T.P^T. MASKED tiles compare each key against
  // the lane's [k_lo, k_hi]; all other tiles run without any mask arithmetic.
  auto tile = [&](const int t, const int buf, auto masked) {
    f32x16 sacc[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) sacc[mb] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const V8 a = *reinterpret_cast<const V8*>(&Ks[buf][mb * 32 + r][16 * kk + 8 * g]);
        sacc[mb] = mfma32(a, qf[kk], sacc[mb]);
      }
    }
    // element (mb, j) holds key t*BN + mb*32 + 8*(j/4) + 4g + j%4
    const int rel_hi = k_hi - (t * BN + 4 * g), rel_lo = k_lo - (t * BN + 4 * g);
    float mloc = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float x = score_value<T, SOFTCAP, REFROUND>(sacc[mb][j], p);
        if constexpr (decltype(masked)::value) {
          const int o = mb * 32 + 8 * (j >> 2) + (j & 3);
          x = (o <= rel_hi && o >= rel_lo) ? x : -INFINITY;
        }
        sacc[mb][j] = x;
        mloc = fmaxf(mloc, x);
      }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
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

    // P = exp2(v*c - m*c), row sums, pack to 16-bit B operands, O^T += V^T . P^T
#pragma unroll
    for (int kk = 0; kk < NPK; ++kk) {
      f32x8 pv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = fast_exp2(fmaf(sacc[kk >> 1][8 * (kk & 1) + e], c, -mc));
        l_part[e & 3] += pe;
        pv[e] = pe;
      }
      const V8 pb = from_f32x8<V8>(pv);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        // A = V^T rows db*32 + r, keys 16kk + 4g + {0..3} and 16kk + 8 + 4g + {0..3} (the P operand's key order),
        // gathered from row-major V by the transposing read (lane m of each 16-lane group points at key row
        // m/4 and head-dim column 4*(m%4) of its 16-column slab).
        const S* vrow = &Vs[buf][16 * kk + 4 * g + tr_krow][db * 32 + tr_dcol];
        const V4 lo = tr_read(vrow);
        const V4 hi = tr_read(vrow + 8 * VP);
        const V8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[db] = mfma32(a, pb, oacc[db]);
      }
    }
  };

  // Tiles [t_begin, t_full0) and [t_full1, t_end) straddle the window's lower edge or the causal diagonal (or the
  // ragged end of K) and evaluate the mask; tiles in between are visible to every row of the workgroup.
  int t_full0 = t_begin, t_full1 = t_end;
  if constexpr (MASK) {
    if (p.window > 0) {  // first tile whose first key is visible to the last row
      const int lo_last = q_last + p.offset - p.window + 1;
      t_full0 = lo_last <= 0 ? t_begin : min(t_end, max(t_begin, (lo_last + BN - 1) / BN));
    }
    if (p.causal) {  // first tile whose last key is hidden from the first row
      const int hi_first = q0 + p.offset;  // last key visible to the first row
      t_full1 = max(t_full0, min(t_end, hi_first < 0 ? t_begin : (hi_first + 1) / BN));
    }
  }
  if (t_full1 > t_full0 && t_full1 * BN > p.Sk) t_full1 = max(t_full0, p.Sk / BN);
  if (t_full1 < t_full0) t_full1 = t_full0;

  // Full next tiles are prefetched into registers before this tile's compute; the ragged last tile (at most one)
  // is loaded after it.
  const bool wave_live = q0 + 32 * w < p.Sq;  // wave-uniform: a wave past the end only stages tiles
  auto step = [&](const int t, auto masked) {
    const int buf = (t - t_begin) & 1;
    const int tn = t + 1;
    const bool prefetch = tn < t_end && tile_full(tn);
    if (prefetch) load_full();
    if (wave_live) tile(t, buf, masked);
    if (tn < t_end) {
      if (!prefetch) load_ragged(tn);
      store_tile(buf ^ 1);
    }
    __syncthreads();
  };
  for (int t = t_begin; t < t_full0; ++t) step(t, std::true_type{});
  for (int t = t_full0; t < t_full1; ++t) step(t, std::false_type{});
  for (int t = t_full1; t < t_end; ++t) step(t, std::true_type{});
  float l_run = (l_part[0] + l_part[1]) + (l_part[2] + l_part[3]);

  // Epilogue: full row sum, normalise, store O (4 consecutive head-dim elements per store) and lse.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = p.Sk == 0 ? 0.f : 1.0f / l_tot;  // no keys at all: o = 0 (an empty P.V), lse = -inf
  if (qi < p.Sq) {
    S* op = static_cast<S*>(p.o) + b * p.o_sb + (int64_t)qi * p.o_ss + h * p.o_sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        V4 ov;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = to_s<S>(oacc[db][4 * jj + e] * inv);
        *reinterpret_cast<V4*>(op + db * 32 + 8 * jj + 4 * g) = ov;
      }
    }
    if (p.lse != nullptr && g == 0) {
      const float lse2 = m_run == -INFINITY ? -INFINITY : m_run * c + fast_log2(l_tot);
      p.lse[(int64_t)bh * p.Sq + qi] = p.lse_base2 ? lse2 : lse2 * kLn2;
    }
  }
}



// ------------------------------------------------------------------------------------------------
// KeyFormer pass 1 (kf.py:36-39): the base-2 log-sum-exp of the Gumbel-perturbed scores of each query row,
//   lse2'[b, h, i] = log2 sum_j exp2(y_ij),  y_ij = (s2_ij - log2 e_ij) / tau,
// over the keys j the row sees, with s2 the score in the exp2 domain (rounded as the reference rounds when
// REFROUND) and e the exp_rand input (gumbels = -log(e), kf.py:37). Four waves of 32 rows; S^T = K.Q^T puts one
// query per lane, so the row reduction stays in the lane (plus one cross-half step). K tiles of 64 keys are staged
// through double-buffered LDS; exp_rand is read once, as 16-byte loads when VEC (rows 16-byte aligned).
// ------------------------------------------------------------------------------------------------
template <typename T, int D, bool MASK, int REFROUND, bool VEC>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) attn_kf_rowlse_kernel(AttnParams p) {
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  constexpr int BN = 64;
  constexpr int KP = D + 8;       // padded K row: 16-byte shift per row for the fragment reads
  constexpr int NKK = D / 16;
  constexpr int NMB = BN / 32;
  constexpr int CPT = BN * D / 8 / kThreads;  // 16-byte chunks per thread per tile
  static_assert(CPT * kThreads == BN * D / 8, "tile mapping");
  __shared__ __attribute__((aligned(16))) S Ks[2][BN][KP];

  int qt, bh;
  map_block(p.n_tiles, p.B * p.Hq, true, qt, bh);
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / p.group;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r = lane & 31, g = lane >> 5;
  const int q0 = qt * kBM;
  const int qi = q0 + 32 * w + r;
  const int qc = min(qi, p.Sq - 1);
  const S* qp = static_cast<const S*>(p.q) + b * p.q_sb + h * p.q_sh;
  const S* kp = static_cast<const S*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const float* erow = p.er + b * p.er_sb + h * p.er_sh + (int64_t)qc * p.er_ss;

  V8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) qf[kk] = ld16<V8>(qp + (int64_t)qc * p.q_ss + 16 * kk + 8 * g);
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    asm volatile("" : "+v"(qf[kk]));
    if (qi >= p.Sq) qf[kk] = V8{};
  }

  const int q_last = min(q0 + kBM, p.Sq) - 1;
  int k_begin = 0, k_end = p.Sk;
  if (p.causal) k_end = min(p.Sk, q_last + p.offset + 1);
  if (p.window > 0) k_begin = max(0, q0 + p.offset - p.window + 1);
  const int t_begin = k_begin / BN;
  const int t_end = k_end > k_begin ? (k_end + BN - 1) / BN : t_begin;
  int k_hi = p.Sk - 1, k_lo = 0;
  if (p.causal) k_hi = min(k_hi, qi + p.offset);
  if (p.window > 0) k_lo = max(k_lo, qi + p.offset - p.window + 1);

  // K staging: copy i of thread tid moves 16-byte chunk (tid + i * kThreads) of the tile, i.e. chunk c % (D/8) of
  // key row c / (D/8) (rows past the end read the last row). Consecutive lanes take consecutive chunks of a row, so
  // each store instruction writes whole rows and the lanes of one LDS pass hit distinct banks (a thread writing
  // CPT adjacent chunks, one instruction per chunk, put lanes 128 bytes apart on the same banks).
  V8 kreg[CPT];
  constexpr int CPR = D / 8;  // chunks per key row
  auto load = [&](int t) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kThreads;
      kreg[i] = ld16<V8>(kp + (int64_t)min(t * BN + c / CPR, p.Sk - 1) * p.k_ss + (c % CPR) * 8);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<V8*>(&Ks[buf][c / CPR][(c % CPR) * 8]) = kreg[i];
    }
  };

  // fp16 reference rounding keeps each pair of scores packed (two instructions per score instead of four)
  constexpr bool PK = REFROUND && std::is_same<T, F16>::value;
  const float cy = (PK ? kLog2e : score_coeff<false, REFROUND>(p)) * p.kf_inv_tau;  // score -> exp2 domain / tau
  f16x2 hpair;
  float m_run = -INFINITY, l_run = 0.f;
  // element (mb, j) of the S^T accumulators holds key t*BN + mb*32 + 8*(j/4) + 4g + j%4. The exp_rand values of
  // tile t+1 are loaded while tile t is computed (ev_next), so the stream stays in flight under the exp/log work.
  f32x4 ev[NMB][4], ev_next[NMB][4];
  // Tiles whose keys all exist (VEC: rows 16-byte aligned) load exp_rand coalesced: load i of lane l reads keys
  // 4 (l % 16) .. +3 of the wave's row 4 i + l / 16, 256 contiguous bytes per row (a load with one row per lane
  // would touch 64 rows, 16 bytes each), and restage() passes the tile through the wave's own LDS rows into the
  // one-row-per-lane layout. Other tiles load that layout directly, 4 bytes at a time.
  constexpr int EV_RS = BN + 4;  // padded LDS row, floats: consecutive rows 4 banks apart
  __shared__ __attribute__((aligned(16))) float Es[kThreads / 64][32 * EV_RS];
  const float* ebase = p.er + b * p.er_sb + h * p.er_sh;
  auto whole = [&](int t) { return VEC && (t + 1) * BN <= p.Sk; };
  auto load_ev = [&](int t, f32x4 (&dst)[NMB][4]) {
    const int kb = t * BN;
    if (whole(t)) {
#pragma unroll
      for (int i = 0; i < 2 * NMB * 2; ++i) {
        const int row = min(q0 + 32 * w + 4 * i + (lane >> 4), p.Sq - 1);
        dst[i >> 2][i & 3] = *reinterpret_cast<const f32x4*>(ebase + (int64_t)row * p.er_ss + kb + 4 * (lane & 15));
      }
      return;
    }
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const int key = kb + mb * 32 + 8 * jq + 4 * g;
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[mb][jq][e] = erow[min(key + e, p.Sk - 1)];
      }
  };
  // The coalesced addressing above (load i: row 4i + lane/16, keys 4*(lane%16)..+3) covers exactly the wave's 32 rows
  // by 64 keys: 2*NMB*2 loads of 4 rows, 16 lanes x 4 keys per row.
  static_assert(BN == 64 && 16 * 4 == BN && 4 * (2 * NMB * 2) == 32, "coalesced exp_rand layout assumes 64-key tiles");
  auto restage = [&](f32x4 (&x)[NMB][4]) {
    float* ew = Es[w];
#pragma unroll
    for (int i = 0; i < 2 * NMB * 2; ++i)
      *reinterpret_cast<f32x4*>(ew + (4 * i + (lane >> 4)) * EV_RS + 4 * (lane & 15)) = x[i >> 2][i & 3];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq)
        x[mb][jq] = *reinterpret_cast<const f32x4*>(ew + r * EV_RS + mb * 32 + 8 * jq + 4 * g);
  };
  auto tile = [&](int t, int buf, auto masked) {
    const int kb = t * BN;
    if (whole(t)) restage(ev);
    f32x16 sacc[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) sacc[mb] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb)
        sacc[mb] = mfma32(*reinterpret_cast<const V8*>(&Ks[buf][mb * 32 + r][16 * kk + 8 * g]), qf[kk], sacc[mb]);
    const int rel_hi = k_hi - (kb + 4 * g), rel_lo = k_lo - (kb + 4 * g);
    float mloc = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        // y = (x2 - log2 e) / tau as one fma of the score against per-launch constants: the score x in the natural
        // log domain times log2(e) / tau (PK: the reference-rounded fp16 pair, read by v_fma_mix), or x * c / tau
        float x;
        if constexpr (PK) {
          if ((j & 1) == 0) hpair = ref_scores_f16(sacc[mb][j], sacc[mb][j + 1], p);
          x = (float)hpair[j & 1];
        } else {
          x = score_value<T, false, REFROUND>(sacc[mb][j], p);
        }
        float y = fmaf(x, cy, -fast_log2(ev[mb][j >> 2][j & 3]) * p.kf_inv_tau);
        if constexpr (decltype(masked)::value) {
          const int o = mb * 32 + 8 * (j >> 2) + (j & 3);
          y = (o <= rel_hi && o >= rel_lo) ? y : -INFINITY;
        }
        sacc[mb][j] = y;
        mloc = fmaxf(mloc, y);
      }
    mloc = half_swap_max(mloc);
    const float m_new = fmaxf(m_run, mloc);
    if (m_new > m_run + kRescaleThreshold || (m_run == -INFINITY && m_new > -INFINITY)) {
      l_run *= fast_exp2(m_run - m_new);  // 0 while m_run is -inf
      m_run = m_new;
    }
    const float mu = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
      for (int j = 0; j < 16; ++j) l_run += fast_exp2(sacc[mb][j] - mu);
  };

  // Tiles [t_full0, t_full1) need no mask for any row of the workgroup (as in attn_fwd_kernel).
  int t_full0 = t_begin, t_full1 = t_end;
  if constexpr (MASK) {
    if (p.window > 0) {
      const int lo_last = q_last + p.offset - p.window + 1;
      t_full0 = lo_last <= 0 ? t_begin : min(t_end, max(t_begin, (lo_last + BN - 1) / BN));
    }
    if (p.causal) {
      const int hi_first = q0 + p.offset;
      t_full1 = max(t_full0, min(t_end, hi_first < 0 ? t_begin : (hi_first + 1) / BN));
    }
  }
  if (t_full1 > t_full0 && t_full1 * BN > p.Sk) t_full1 = max(t_full0, p.Sk / BN);
  if (t_full1 < t_full0) t_full1 = t_full0;

  if (t_begin < t_end) {
    load(t_begin);
    load_ev(t_begin, ev);
    store(0);
  }
  __syncthreads();
  auto step = [&](int t, auto masked) {
    const int buf = (t - t_begin) & 1;
    const bool more = t + 1 < t_end;
    if (more) {
      load(t + 1);
      load_ev(t + 1, ev_next);
    }
    tile(t, buf, masked);
    if (more) store(buf ^ 1);
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) ev[mb][jq] = ev_next[mb][jq];
  };
  for (int t = t_begin; t < t_full0; ++t) step(t, std::true_type{});
  for (int t = t_full0; t < t_full1; ++t) step(t, std::false_type{});
  for (int t = t_full1; t < t_end; ++t) step(t, std::true_type{});

  const float l_tot = half_swap_sum(l_run);
  if (qi < p.Sq && g == 0) p.lse[(int64_t)bh * p.Sq + qi] = m_run == -INFINITY ? -INFINITY : m_run + fast_log2(l_tot);
}

// NQB: 32-row query blocks per wave (each K / V fragment feeds NQB MFMAs); NW: waves per workgroup; BN: keys
// per tile; NSTAGE: tiles in the LDS ring; OCC: waves per SIMD the register budget is sized for. FASTSUM: the row
// sums add the 16-bit rounded probabilities two at a time (v_dot2); used when no lse is written, since the O
// normalisation tolerates the rounding but the column-sum pass needs the fp32 row sums.
template <typename T, int D, int NQB, int NW, int BN, int NSTAGE, int OCC, bool MASK, bool SOFTCAP, int REFROUND,
          bool FASTSUM>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
attn_fwd_dma_kernel(AttnParams p) {
  typedef DmaLayout<D> L;
  constexpr int ROW_B = L::ROW_B, GROUP_B = L::GROUP_B, LPR = L::LPR, RPI = L::RPI, IPG = L::IPG;
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  typedef typename T::vec4 V4;
  constexpr int QPW = 32 * NQB;                 // query rows per wave
  constexpr int BM = QPW * NW;                  // query rows per workgroup
  constexpr int TILE_B = (BN / 4) * GROUP_B;
  constexpr int STAGE_B = 2 * TILE_B;           // K tile, then V tile
  constexpr int GPW = (BN / 4) / NW;            // 4-row groups of a tile copied by each wave (K and V each)
  constexpr int DMA_PER_TILE = 2 * GPW * IPG;   // direct loads per wave per tile
  static_assert(GPW >= 1 && GPW * NW == BN / 4, "tile groups must split over the waves");
  __shared__ __attribute__((aligned(1024))) char smem[NSTAGE * STAGE_B];

  int qt, bh;
  map_block_kv(p.n_tiles, p.B, p.Hq, p.Hkv, true, qt, bh);
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / p.group;
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qt * BM;
  const int qw0 = q0 + QPW * w;  // first query row of this wave; lane rows qw0 + 32n + r, n = 0, 1

  const S* qp = static_cast<const S*>(p.q) + b * p.q_sb + h * p.q_sh;
  const char* kp = reinterpret_cast<const char*>(static_cast<const S*>(p.k) + b * p.k_sb + hk * p.k_sh);
  const char* vp = reinterpret_cast<const char*>(static_cast<const S*>(p.v) + b * p.v_sb + hk * p.v_sh);
  const int64_t k_ss_b = p.k_ss * (int64_t)sizeof(S), v_ss_b = p.v_ss * (int64_t)sizeof(S);

  // Q fragments: all loads issued back to back (rows past the end read the last row and are zeroed afterwards;
  // a load under a per-row branch would be waited for on its own).
  V8 qf[NQB][D / 16];
#pragma unroll
  for (int n = 0; n < NQB; ++n) {
    const int qi = min(qw0 + 32 * n + r, p.Sq - 1);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) qf[n][kk] = ld16<V8>(qp + (int64_t)qi * p.q_ss + 16 * kk + 8 * g);
  }
  // Fused rotary of the query (head_dim 128): the (cos, sin) of this lane's 32 rotary pairs, loaded with Q so that
  // the two latencies overlap. The lane holds elements 16kk + 8g + e of fragment kk and their pair partners (+64)
  // in fragment kk + 4, so it rotates its own pairs.
  constexpr int NRC = D == 128 ? NQB : 0;
  f32x8 rcos[NRC > 0 ? NRC : 1][4], rsin[NRC > 0 ? NRC : 1][4];
  const bool rope = D == 128 && p.rope_cs != nullptr;
  if constexpr (NRC > 0) {
    if (rope) {
#pragma unroll
      for (int n = 0; n < NQB; ++n) {
        const float* cs = p.rope_cs + ((int64_t)b * p.Sq + min(qw0 + 32 * n + r, p.Sq - 1)) * D + 8 * g;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          rcos[n][kk] = *reinterpret_cast<const f32x8*>(cs + 16 * kk);
          rsin[n][kk] = *reinterpret_cast<const f32x8*>(cs + 64 + 16 * kk);
        }
      }
    }
  }
  // BIAS (bf16 without soft-cap or reference rounding, no lse): Q is pre-scaled by scale*log2(e) and each score
  // accumulator starts from -m (the row's reference maximum) through one extra MFMA whose A fragment is the
  // constant column e_0 and whose B fragment holds -m in k-slot 0. The accumulator then holds s*c - m and
  // P = exp2(acc) needs no per-element arithmetic. The reference maxima are bf16 values so that -m is exact in
  // the B operand; the pre-scaled Q carries the same 2^-9 relative rounding as the reference's bf16 scores.
  constexpr bool BIAS = FASTSUM && !SOFTCAP && !REFROUND && std::is_same<T, BF16>::value;
  // Waits for the Q loads (after the first K / V copies are issued, so that the latencies overlap), zeroes rows
  // past the end, pre-scales for BIAS and pins the fragments in registers: AGPRs at one wave per SIMD (head_dim
  // 256: MFMA reads its B operand from there, the VGPRs stay free for the scores and the fragments read ahead).
  auto finish_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < NQB; ++n) {
      const bool live = qw0 + 32 * n + r < p.Sq;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) asm volatile("" : "+v"(qf[n][kk]));
      if constexpr (NRC > 0) {
        // pos_encoding.cu:90-112 on this lane's row: rotated in fp32, rounded to the storage type as the rotary
        // kernel stores it
        if (rope) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const f32x8 c = rcos[n][kk], sn = rsin[n][kk];
            const f32x8 x = to_f32x8(qf[n][kk]), y = to_f32x8(qf[n][kk + 4]);
            f32x8 xo, yo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              xo[e] = x[e] * c[e] - y[e] * sn[e];
              yo[e] = y[e] * c[e] + x[e] * sn[e];
            }
            qf[n][kk] = from_f32x8<V8>(xo);
            qf[n][kk + 4] = from_f32x8<V8>(yo);
          }
        }
      }
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        if (!live) qf[n][kk] = V8{};
        if constexpr (BIAS) qf[n][kk] = from_f32x8<V8>(to_f32x8(qf[n][kk]) * p.c_fast);
        if constexpr (OCC == 1) asm volatile("" : "+a"(qf[n][kk]));
        else asm volatile("" : "+v"(qf[n][kk]));
      }
    }
  };
  V8 abias = V8{};
  abias[0] = g == 0 ? to_s<S>(1.0f) : to_s<S>(0.0f);
  V8 bbias[NQB];
#pragma unroll
  for (int n = 0; n < NQB; ++n) bbias[n] = V8{};

  // Key tiles of the workgroup and of this wave.
  const int q_last = min(q0 + BM, p.Sq) - 1;
  int k_begin = 0, k_end = p.Sk;
  if (p.causal) k_end = min(p.Sk, q_last + p.offset + 1);
  if (p.window > 0) k_begin = max(0, q0 + p.offset - p.window + 1);
  const int t_begin = k_begin / BN;
  const int t_end = k_end > k_begin ? (k_end + BN - 1) / BN : t_begin;
  const int wq_last = min(qw0 + QPW, p.Sq) - 1;  // may be < qw0 for a wave past the end
  int wk_begin = 0, wk_end = p.Sk;
  if (p.causal) wk_end = min(p.Sk, wq_last + p.offset + 1);
  if (p.window > 0) wk_begin = max(0, qw0 + p.offset - p.window + 1);

  // Visible keys per lane row: lo <= key <= hi.
  int k_hi[NQB], k_lo[NQB];
#pragma unroll
  for (int n = 0; n < NQB; ++n) {
    const int qi = qw0 + 32 * n + r;
    k_hi[n] = p.Sk - 1;
    k_lo[n] = 0;
    if (p.causal) k_hi[n] = min(k_hi[n], qi + p.offset);
    if (p.window > 0) k_lo[n] = max(k_lo[n], qi + p.offset - p.window + 1);
  }

  // Direct-load lane constants: in load i of a 4-row group, lane l fills LDS position l%LPR of group row
  // i*RPI + l/LPR, fetching global chunk (l%LPR) ^ 4*(group row).
  uint32_t src_chunk[IPG], k_voff[IPG], v_voff[IPG];
#pragma unroll
  for (int i = 0; i < IPG; ++i) {
    const int grow = i * RPI + lane / LPR;
    src_chunk[i] = (uint32_t)((lane % LPR) ^ (grow << 2));
    k_voff[i] = (uint32_t)(grow * k_ss_b) + src_chunk[i] * 16u;
    v_voff[i] = (uint32_t)(grow * v_ss_b) + src_chunk[i] * 16u;
    asm volatile("" : "+v"(k_voff[i]), "+v"(v_voff[i]));
  }
  const uint32_t smem_base = (uint32_t)(size_t)((lds_char*)smem);

  // Copies groups GPW*w .. GPW*w + GPW-1 of tile t into stage t % NSTAGE: DMA_PER_TILE loads per wave.
  auto issue = [&](int t) {
    const uint32_t kdst = smem_base + (uint32_t)((t % NSTAGE) * STAGE_B + GPW * w * GROUP_B);
    const uint32_t vdst = kdst + TILE_B;
    const int row0 = t * BN + 4 * GPW * w;
    if ((t + 1) * BN <= p.Sk) {
      const char* kb = kp + (int64_t)row0 * k_ss_b;
      const char* vb = vp + (int64_t)row0 * v_ss_b;
#pragma unroll
      for (int j = 0; j < GPW; ++j)
#pragma unroll
        for (int i = 0; i < IPG; ++i) {
          dma16(kdst + j * GROUP_B + i * RPI * ROW_B, kb + 4 * j * k_ss_b, k_voff[i]);
          dma16(vdst + j * GROUP_B + i * RPI * ROW_B, vb + 4 * j * v_ss_b, v_voff[i]);
        }
    } else {  // ragged last tile: rows past the end re-read the last row (always masked, finite)
#pragma unroll
      for (int j = 0; j < GPW; ++j)
#pragma unroll
        for (int i = 0; i < IPG; ++i) {
          const int64_t row = min(row0 + 4 * j + i * RPI + lane / LPR, p.Sk - 1);
          dma16(kdst + j * GROUP_B + i * RPI * ROW_B, kp + row * k_ss_b + src_chunk[i] * 16);
          dma16(vdst + j * GROUP_B + i * RPI * ROW_B, vp + row * v_ss_b + src_chunk[i] * 16);
        }
    }
  };

  // Load i (0 .. DMA_PER_TILE-1) of issue(t) for a tile whose rows all exist: the K loads, then the V loads. The
  // mask-free tiles issue the next tile's copies one per QK^T step with these, so that the copies' issue overlaps
  // the MFMAs instead of following the barrier as one burst (which held every wave of the workgroup at once).
  auto issue_one = [&](int t, int i) __attribute__((always_inline)) {
    const uint32_t kdst = smem_base + (uint32_t)((t % NSTAGE) * STAGE_B + GPW * w * GROUP_B);
    const int row0 = t * BN + 4 * GPW * w;
    const int half = GPW * IPG, ii = i % half, j = ii / IPG, l = ii % IPG;
    if (i < half)
      dma16(kdst + j * GROUP_B + l * RPI * ROW_B, kp + (int64_t)row0 * k_ss_b + 4 * j * k_ss_b, k_voff[l]);
    else
      dma16(kdst + TILE_B + j * GROUP_B + l * RPI * ROW_B, vp + (int64_t)row0 * v_ss_b + 4 * j * v_ss_b, v_voff[l]);
  };
  static_assert(DMA_PER_TILE <= D / 16, "one copy per QK^T step");

  // LDS read addressing. K fragment (row mb*32 + r, chunk 2kk + g): lane part + xk[kk/2] + constant.
  // V transposing read (rows 16kk + 4g + (lane%16)/4 (+8), head-dim column db*32 + 16*((lane/16)%2) + 4*(lane%4)):
  // lane part + xv[db] + constant.
  const int s4 = r & 3;
  const uint32_t k_lane = (uint32_t)((r >> 2) * GROUP_B + s4 * ROW_B + 16 * g);
  uint32_t xk[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) xk[i] = k_lane + 64u * (uint32_t)(i ^ s4);
  const int m4 = (lane & 15) >> 2, m3 = lane & 3;
  const uint32_t v_lane = (uint32_t)(TILE_B + g * GROUP_B + m4 * ROW_B + 32 * ((lane >> 4) & 1) + 16 * (m3 >> 1) +
                                     8 * (m3 & 1));
  uint32_t xv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) xv[db] = v_lane + 64u * (uint32_t)(db ^ m4);

  f32x16 oacc[NQB][D / 32];
  float m_run[NQB], l_part[NQB][2];
#pragma unroll
  for (int n = 0; n < NQB; ++n) {
#pragma unroll
    for (int i = 0; i < D / 32; ++i) oacc[n][i] = f32x16{};
    m_run[n] = -INFINITY;
    l_part[n][0] = l_part[n][1] = 0.f;
  }
  // fp16 reference rounding without soft-cap keeps the scores as packed fp16 in the natural-log domain.
  constexpr bool PK = REFROUND && !SOFTCAP && std::is_same<T, F16>::value;
  const float c = PK ? kLog2e : score_coeff<SOFTCAP, REFROUND>(p);

  // SPREAD (mask-free tiles): the copies of tile t + NSTAGE - 1 are issued here, one per QK^T step.
  auto tile = [&](const int t, auto masked) {
    constexpr bool SPREAD = !decltype(masked)::value && DGG_SPREAD_COPIES;
    const uint32_t st = smem_base + (uint32_t)((t % NSTAGE) * STAGE_B);
    // Per-stage base addresses, opaque to the compiler so that every fragment read below is base + immediate
    // offset (otherwise it re-adds the stage offset for each read).
    uint32_t kbase[D / 32], vbase[D / 32];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      kbase[i] = st + xk[i];
      vbase[i] = st + xv[i];
      asm volatile("" : "+v"(kbase[i]), "+v"(vbase[i]));
    }
    constexpr int NMB = BN / 32;
    constexpr bool MASKED = decltype(masked)::value;
    // Masked tiles: per 32-key block, whether any of the wave's rows sees any of its keys (live) and whether every
    // row sees every key (full). Dead blocks skip their MFMAs and exps, full blocks the per-element mask.
    bool blk_live[NMB], blk_full[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) blk_live[mb] = blk_full[mb] = true;
    if constexpr (MASKED) {
      const int row_hi = max(qw0, min(qw0 + QPW, p.Sq) - 1);
      const int hi_min = p.causal ? min(p.Sk - 1, qw0 + p.offset) : p.Sk - 1;
      const int hi_max = p.causal ? min(p.Sk - 1, row_hi + p.offset) : p.Sk - 1;
      const int lo_min = p.window > 0 ? max(0, qw0 + p.offset - p.window + 1) : 0;
      const int lo_max = p.window > 0 ? max(0, row_hi + p.offset - p.window + 1) : 0;
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const int kb0 = t * BN + mb * 32;
        blk_live[mb] = kb0 <= hi_max && kb0 + 31 >= lo_min;
        blk_full[mb] = kb0 >= lo_max && kb0 + 31 <= hi_min;
      }
    }
    f32x16 sacc[NQB][NMB];
#pragma unroll
    for (int n = 0; n < NQB; ++n)
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        if constexpr (BIAS) sacc[n][mb] = mfma32(abias, bbias[n], f32x16{});  // every element = -m[n]
        else sacc[n][mb] = f32x16{};
      }
    if constexpr (MASKED) {
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        if (!blk_live[mb]) continue;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const V8 a = lds_read<V8>(kbase[kk >> 1] + mb * 8 * GROUP_B + 32 * (kk & 1));
#pragma unroll
          for (int n = 0; n < NQB; ++n) sacc[n][mb] = mfma32(a, qf[n][kk], sacc[n][mb]);
        }
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        if constexpr (SPREAD) {
          if (kk < DMA_PER_TILE) issue_one(t + NSTAGE - 1, kk);
        }
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
          const V8 a = lds_read<V8>(kbase[kk >> 1] + mb * 8 * GROUP_B + 32 * (kk & 1));
#pragma unroll
          for (int n = 0; n < NQB; ++n) sacc[n][mb] = mfma32(a, qf[n][kk], sacc[n][mb]);
        }
      }
    }
    const int kb4 = t * BN + 4 * g;
    constexpr bool PKM = PK && !decltype(masked)::value;  // scores stay packed fp16 through the P stage
    f16x2 hs[NQB][NMB][8];
#pragma unroll
    for (int n = 0; n < NQB; ++n) {
      const int rel_hi = k_hi[n] - kb4, rel_lo = k_lo[n] - kb4;
      float mloc = -INFINITY;
      if constexpr (PK) {
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int jp = 0; jp < 8; ++jp) hs[n][mb][jp] = ref_scores_f16(sacc[n][mb][2 * jp], sacc[n][mb][2 * jp + 1], p);
      }
      if constexpr (PKM) {
        f16x2 mx = hs[n][0][0];
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int jp = 0; jp < 8; ++jp) mx = __builtin_elementwise_max(mx, hs[n][mb][jp]);
        mloc = fmaxf((float)mx[0], (float)mx[1]);
      } else {
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            float x;
            if constexpr (PK) x = (float)hs[n][mb][j >> 1][j & 1];
            else x = score_value<T, SOFTCAP, REFROUND>(sacc[n][mb][j], p);
            if constexpr (MASKED) {
              const int o = mb * 32 + 8 * (j >> 2) + (j & 3);
              if (!blk_live[mb]) x = -INFINITY;
              else if (!blk_full[mb]) x = (o <= rel_hi && o >= rel_lo) ? x : -INFINITY;
            }
            sacc[n][mb][j] = x;
            mloc = fmaxf(mloc, x);
          }
        }
      }
      mloc = half_swap_max(mloc);
      if constexpr (BIAS) {
        // mloc is relative to m_run (or absolute while m_run is still -inf and the bias is 0)
        const bool first = m_run[n] == -INFINITY;
        const bool need = first ? mloc > -INFINITY : mloc > kRescaleThreshold;
        if (__any(need)) {
          const float base = first ? 0.f : m_run[n];
          const float m_new = need ? to_f(to_s<S>(mloc + base)) : m_run[n];
          const float alpha = need ? fast_exp2(m_run[n] - m_new) : 1.0f;
          const float delta = need ? m_new - base : 0.f;
          m_run[n] = m_new;
          bbias[n][0] = g == 0 && m_new != -INFINITY ? to_s<S>(-m_new) : to_s<S>(0.0f);
          l_part[n][0] *= alpha;
          l_part[n][1] *= alpha;
#pragma unroll
          for (int i = 0; i < D / 32; ++i) oacc[n][i] *= alpha;
#pragma unroll
          for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int j = 0; j < 16; ++j) sacc[n][mb][j] -= delta;
        }
        continue;
      }
      const float m_new = fmaxf(m_run[n], mloc);
      const bool need = m_new * c > m_run[n] * c + kRescaleThreshold;
      if (__any(need)) {
        const float alpha = need ? fast_exp2((m_run[n] - m_new) * c) : 1.0f;
        if (need) m_run[n] = m_new;
        l_part[n][0] *= alpha;
        l_part[n][1] *= alpha;
#pragma unroll
        for (int i = 0; i < D / 32; ++i) oacc[n][i] *= alpha;
      }
    }
    float mcs[NQB];
#pragma unroll
    for (int n = 0; n < NQB; ++n) mcs[n] = BIAS || m_run[n] == -INFINITY ? 0.f : m_run[n] * c;
#pragma unroll
    for (int kk = 0; kk < BN / 16; ++kk) {
      if (MASKED && !blk_live[kk >> 1]) continue;  // P = 0 there
      V8 pb[NQB];
#pragma unroll
      for (int n = 0; n < NQB; ++n) {
        const float mc = mcs[n];
        f32x8 pv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float x;
          if constexpr (PKM) x = (float)hs[n][kk >> 1][4 * (kk & 1) + (e >> 1)][e & 1];
          else x = sacc[n][kk >> 1][8 * (kk & 1) + e];
          const float pe = BIAS ? fast_exp2(x) : fast_exp2(fmaf(x, c, -mc));
          if constexpr (!FASTSUM) l_part[n][e & 1] += pe;
          pv[e] = pe;
        }
        pb[n] = from_f32x8<V8>(pv);
        if constexpr (FASTSUM) l_part[n][kk & 1] = rowsum8(pb[n], l_part[n][kk & 1]);
      }
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const V4 lo = tr_read_at(vbase[db] + kk * 4 * GROUP_B, S{});
        const V4 hi = tr_read_at(vbase[db] + kk * 4 * GROUP_B + 2 * GROUP_B, S{});
        const V8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int n = 0; n < NQB; ++n) oacc[n][db] = mfma32(a, pb[n], oacc[n][db]);
      }
    }
  };

  // Tile classes, as in the generic kernel but per wave: tiles outside [wk_begin, wk_end) are skipped by this
  // wave (it still takes part in the loads and barriers); [t_full0, t_full1) needs no mask for any of its rows.
  int t_full0 = t_begin, t_full1 = t_end;
  if constexpr (MASK) {
    if (p.window > 0) {
      const int lo_last = wq_last + p.offset - p.window + 1;
      t_full0 = lo_last <= 0 ? t_begin : min(t_end, max(t_begin, (lo_last + BN - 1) / BN));
    }
    if (p.causal) {
      const int hi_first = qw0 + p.offset;
      t_full1 = max(t_full0, min(t_end, hi_first < 0 ? t_begin : (hi_first + 1) / BN));
    }
  }
  if (t_full1 > t_full0 && t_full1 * BN > p.Sk) t_full1 = max(t_full0, p.Sk / BN);
  if (t_full1 < t_full0) t_full1 = t_full0;
  // A wave whose rows all lie past the end (qw0 >= Sq: the last workgroup of a ragged or short query range,
  // e.g. a single decode-like row) computes no tile; it still issues its share of the copies and meets the barriers.
  const int wt_begin = wk_begin / BN;
  const int wt_end = qw0 < p.Sq && wk_end > wk_begin ? (wk_end + BN - 1) / BN : wt_begin;

  // Pipeline: tiles t+1 .. t+NSTAGE-2 may still be in flight while tile t is waited for; the copy of tile
  // t+NSTAGE-1 is issued after the barrier into the stage that held tile t-1.
#pragma unroll
  for (int i = 0; i < NSTAGE - 1; ++i)
    if (t_begin + i < t_end) issue(t_begin + i);
  finish_q();
  auto step = [&](const int t, auto masked) {
    const int after = min(NSTAGE - 2, t_end - 1 - t);
    if (NSTAGE >= 4 && after >= 2) wait_vmem<2 * DMA_PER_TILE>();
    else if (NSTAGE >= 3 && after >= 1) wait_vmem<DMA_PER_TILE>();
    else wait_vmem<0>();
    __syncthreads();
    constexpr bool SPREAD = !decltype(masked)::value && DGG_SPREAD_COPIES;
    if (!SPREAD && t + NSTAGE - 1 < t_end) issue(t + NSTAGE - 1);
    if (SPREAD || (t >= wt_begin && t < wt_end)) tile(t, masked);
  };
  // Mask-free steps issue their copies inside the tile, so they are the tiles this wave computes whose copy target
  // t + NSTAGE - 1 exists and is whole; the others (at most NSTAGE - 1 of them) take the masked step, which is
  // correct for any tile.
  int t_sp1 = t_full1;
  if (DGG_SPREAD_COPIES) t_sp1 = min(min(t_full1, wt_end), min(t_end, p.Sk / BN) - (NSTAGE - 1));
  const int t_sp0 = DGG_SPREAD_COPIES ? min(max(t_full0, wt_begin), t_end) : t_full0;
  t_sp1 = max(t_sp0, t_sp1);
  for (int t = t_begin; t < t_sp0; ++t) step(t, std::true_type{});
  for (int t = t_sp0; t < t_sp1; ++t) step(t, std::false_type{});
  for (int t = t_sp1; t < t_end; ++t) step(t, std::true_type{});

#pragma unroll
  for (int n = 0; n < NQB; ++n) {
    const int qi = qw0 + 32 * n + r;
    const float l_tot = half_swap_sum(l_part[n][0] + l_part[n][1]);
    const float inv = p.Sk == 0 ? 0.f : 1.0f / l_tot;  // no keys at all: o = 0 (an empty P.V), lse = -inf
    if (qi < p.Sq) {
      S* op = static_cast<S*>(p.o) + b * p.o_sb + (int64_t)qi * p.o_ss + h * p.o_sh;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          V4 ov;
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[e] = to_s<S>(oacc[n][db][4 * jj + e] * inv);
          *reinterpret_cast<V4*>(op + db * 32 + 8 * jj + 4 * g) = ov;
        }
      }
      if (p.lse != nullptr && g == 0) {
        const float lse2 = m_run[n] == -INFINITY ? -INFINITY : m_run[n] * c + fast_log2(l_tot);
        p.lse[(int64_t)bh * p.Sq + qi] = p.lse_base2 ? lse2 : lse2 * kLn2;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Column-sum kernel: colsum[b,h,j] = sum_i exp(score_ij - lse_i). A workgroup owns 128 keys (32 per wave,
// held in VGPRs as the B operand); query tiles of 64 rows stream through double-buffered LDS together
// with their lse. S (64 x 32) = Q . K^T puts one key per lane, so each lane sums its own column.
// ------------------------------------------------------------------------------------------------
constexpr int kCBQ = 64;   // query rows per tile
constexpr int kCBK = 32 * kWaves;  // keys per workgroup

template <typename T, int D, bool MASK, bool SOFTCAP, int REFROUND, int EPI>
__global__ void __launch_bounds__(kThreads) attn_colsum_kernel(AttnParams p) {
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  constexpr int QP = D + 8;
  constexpr int NKK = D / 16;
  constexpr int NMB = kCBQ / 32;
  constexpr int CHUNKS = kCBQ * D / 8;
  constexpr int CPT = (CHUNKS + kThreads - 1) / kThreads;

  __shared__ __attribute__((aligned(16))) S Qs[2][kCBQ][QP];
  __shared__ float Ls[2][kCBQ];

  int kt, bh;
  map_block(p.n_tiles, p.B * p.Hq, false, kt, bh);
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / p.group;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r = lane & 31, g = lane >> 5;
  const int k0 = kt * kCBK;
  const int kj = k0 + 32 * w + r;  // this lane's key

  const S* qp = static_cast<const S*>(p.q) + b * p.q_sb + h * p.q_sh;
  const S* kp = static_cast<const S*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const float* lsep = p.lse + (int64_t)bh * p.Sq;

  V8 kf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)  // back-to-back loads (keys past the end read the last key, zeroed below)
    kf[kk] = ld16<V8>(kp + (int64_t)min(kj, p.Sk - 1) * p.k_ss + 16 * kk + 8 * g);
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    asm volatile("" : "+v"(kf[kk]));  // see the forward kernel
    if (kj >= p.Sk) kf[kk] = V8{};
  }

  // Query range that can see any key of this tile.
  const int k_last = min(k0 + kCBK, p.Sk) - 1;
  int q_begin = 0, q_end = p.Sq;
  if (p.causal) q_begin = max(0, k0 - p.offset);
  if (p.window > 0) q_end = min(p.Sq, k_last - p.offset + p.window);
  const int t_begin = q_begin / kCBQ;
  const int t_end = q_end > q_begin ? (q_end + kCBQ - 1) / kCBQ : t_begin;
  const float c = score_coeff<SOFTCAP, REFROUND>(p);

  V8 qreg[CPT];
  float lreg = 0.f;
  auto load_tile = [&](int t) {
    const int qb = t * kCBQ;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = tid + i * kThreads;
      if (CHUNKS % kThreads == 0 || ch < CHUNKS) {
        const int row = ch / (D / 8), dc = ch % (D / 8);
        const int qg = qb + row;
        qreg[i] = qg < p.Sq ? ld16<V8>(qp + (int64_t)qg * p.q_ss + dc * 8) : V8{};
      }
    }
    if (tid < kCBQ) {
      const int qg = qb + tid;
      // Rows past the end get +inf so that their probability is exp2(-inf) = 0.
      lreg = qg < p.Sq ? (p.lse_base2 ? lsep[qg] : lsep[qg] * kLog2e) : INFINITY;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = tid + i * kThreads;
      if (CHUNKS % kThreads == 0 || ch < CHUNKS) {
        const int row = ch / (D / 8), dc = ch % (D / 8);
        *reinterpret_cast<V8*>(&Qs[buf][row][dc * 8]) = qreg[i];
      }
    }
    if (tid < kCBQ) Ls[buf][tid] = lreg;
  };

  if (t_begin < t_end) {
    load_tile(t_begin);
    store_tile(0);
  }
  __syncthreads();

  ColAcc<EPI> acc;
  const int kjc = min(kj, p.Sk - 1);
  const float* erp = EPI == kColKF ? p.er + b * p.er_sb + h * p.er_sh : nullptr;  // KeyFormer exp_rand of (b, h)
  for (int t = t_begin; t < t_end; ++t) {
    const int buf = (t - t_begin) & 1;
    const bool has_next = t + 1 < t_end;
    if (has_next) load_tile(t + 1);

    f32x16 sacc[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) sacc[mb] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const V8 a = *reinterpret_cast<const V8*>(&Qs[buf][mb * 32 + r][16 * kk + 8 * g]);
        sacc[mb] = mfma32(a, kf[kk], sacc[mb]);
      }
    }

    const int qb = t * kCBQ;
    bool need_mask = qb + kCBQ > p.Sq || k0 + kCBK > p.Sk;
    if constexpr (MASK) {
      if (p.causal && qb + p.offset < k_last) need_mask = true;
      if (p.window > 0 && qb + kCBQ - 1 + p.offset - k0 >= p.window) need_mask = true;
    }
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int row = mb * 32 + 8 * (j >> 2) + 4 * g + (j & 3);
        const float x = score_value<T, SOFTCAP, REFROUND>(sacc[mb][j], p);
        const int qg = qb + row;
        float pe;
        if constexpr (EPI == kColKF)
          pe = kf_prob(x * c, erp[(int64_t)min(qg, p.Sq - 1) * p.er_ss + kjc], Ls[buf][row], p);
        else
          pe = fast_exp2(fmaf(x, c, -Ls[buf][row]));
        bool vis = true;  // (qg, kj) a visible pair of an existing row and key
        if (need_mask) {
          bool ok = qg < p.Sq && kj < p.Sk;
          if constexpr (MASK) {
            const int rel = qg + p.offset - kj;
            if (p.causal) ok = ok && rel >= 0;
            if (p.window > 0) ok = ok && rel < p.window;
          }
          pe = ok ? pe : 0.f;
          vis = ok;
        }
        // Corm compares visible pairs here; the masked ones (p = 0) are ORed in by corm_masked_or_kernel
        acc.add(pe, EPI == kColAnyGe ? vis : qg < p.Sq, min(qg, p.Sq - 1), kjc, p);
      }
    }

    if (has_next) store_tile(buf ^ 1);
    __syncthreads();
  }
  acc.store(p, bh, kj, g);
}

// ------------------------------------------------------------------------------------------------
// Column-sum kernel for head_dim 128. A workgroup of NW waves owns 32*NW keys; wave w keeps keys
// k0 + 32w .. + 31 in VGPRs as the B operand. Query tiles of BQ rows stream through an NSTAGE ring in LDS
// with the forward's swizzled layout and direct-to-LDS copies (the Q tile takes the place of the K tile),
// each stage followed by the BQ lse values of its rows (global_load_lds_dword, issued by the last wave).
// S (BQ x 32) = Q . K^T puts one key per lane: accumulator register j of block mb holds query row
// 32mb + 8(j/4) + 4(lane/32) + j%4, so each lane sums its key's column over its rows, and the partner
// lane (lane ^ 32) adds the other half at the end.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ void dma4(uint32_t lds, const void* vaddr) {
  // lane l's 4 bytes land at LDS byte address lds + 4*l (lanes switched off by EXEC write nothing)
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(vaddr)
               : "memory", "m0");
}

// KPW: 32-key blocks per wave. With two, each Q fragment read from the LDS feeds two MFMAs (one per key block).
template <typename T, int NW, int KPW, int BQ, int NSTAGE, bool MASK, bool SOFTCAP, int REFROUND, bool LSE2, int EPI>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_colsum_d128_kernel(AttnParams p) {
  constexpr int D = 128;
  constexpr int ROW_B = DmaLayout<D>::ROW_B, GROUP_B = DmaLayout<D>::GROUP_B;
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  // With KPW key blocks per wave the waves form KPW row groups of NW / KPW waves: each group covers every key of
  // the workgroup and takes its own BQ / KPW rows of each query tile; the groups' sums are added at the end.
  constexpr int NG = KPW, NWG = NW / NG;     // row groups, waves per group
  constexpr int BQW = BQ / NG;               // query rows of a tile per row group
  constexpr int BK = 32 * KPW * NWG;         // keys per workgroup
  constexpr int QT_B = (BQ / 4) * GROUP_B;   // bytes of one Q tile
  constexpr int STAGE_B = QT_B + 4 * BQ;     // Q tile, then its BQ lse values
  constexpr int GPW = (BQ / 4) / NW;         // 4-row groups of a Q tile copied by each wave
  constexpr int NLSE = BQ / 64;              // lse copies per tile (last wave only)
  constexpr int NMB = BQW / 32;              // 32-row query blocks of a wave's part of a tile
  static_assert(GPW >= 1 && GPW * NW == BQ / 4, "Q tile groups must split over the waves");
  static_assert(BQ % 64 == 0 && QT_B % 16 == 0 && BQW % 32 == 0 && NWG * NG == NW, "tile shape");
  static_assert(KPW == 1 || ((EPI == kColSum || EPI == kColSumSq) && KPW == 2), "two key blocks: sum epilogues");
  static_assert(NG == 1 || NSTAGE * STAGE_B >= 4 * 2 * BK, "the groups' sums are combined in the LDS");
  constexpr int NSB = KPW * NMB;  // score blocks of a tile: block kp * NMB + mb (key block kp, query block mb)
  __shared__ __attribute__((aligned(1024))) char smem[NSTAGE * STAGE_B];

  int kt, bh;
  map_block(p.n_tiles, p.B * p.Hq, false, kt, bh);
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / p.group;
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wi = w % NWG, gw = w / NWG;  // wave within its row group, row group
  const int rg0 = BQW * gw;              // first row of the group's part of a query tile
  const int k0 = kt * BK;
  const int kw0 = k0 + 32 * KPW * wi;  // first key of this wave
  const int kj = kw0 + r;             // this lane's key (of key block 0; block kp: kj + 32 kp)

  const S* kp = static_cast<const S*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const char* qp = reinterpret_cast<const char*>(static_cast<const S*>(p.q) + b * p.q_sb + h * p.q_sh);
  const int64_t q_ss_b = p.q_ss * (int64_t)sizeof(S);
  const float* lsep = p.lse + (int64_t)bh * p.Sq;

  V8 kf[KPW][D / 16];
#pragma unroll
  for (int kb = 0; kb < KPW; ++kb)
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)  // back-to-back loads (keys past the end read the last key, zeroed below)
      kf[kb][kk] = ld16<V8>(kp + (int64_t)min(kj + 32 * kb, p.Sk - 1) * p.k_ss + 16 * kk + 8 * g);
#pragma unroll
  for (int kb = 0; kb < KPW; ++kb)
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      asm volatile("" : "+v"(kf[kb][kk]));  // see the forward kernel
      if (kj + 32 * kb >= p.Sk) kf[kb][kk] = V8{};
    }

  // Query tiles that see any key of the workgroup, and of this wave.
  const int k_last = min(k0 + BK, p.Sk) - 1;
  int q_begin = 0, q_end = p.Sq;
  if (p.causal) q_begin = max(0, k0 - p.offset);
  if (p.window > 0) q_end = min(p.Sq, k_last - p.offset + p.window);
  const int t_begin = q_begin / BQ;
  const int t_end = q_end > q_begin ? (q_end + BQ - 1) / BQ : t_begin;
  int wt_begin = t_begin, wt_end = t_begin;  // empty for a wave whose keys all lie past Sk
  if (kw0 < p.Sk) {
    const int wk_last = min(kw0 + 32 * KPW, p.Sk) - 1;
    int wq_begin = 0, wq_end = p.Sq;
    if (p.causal) wq_begin = max(0, kw0 - p.offset);
    if (p.window > 0) wq_end = min(p.Sq, wk_last - p.offset + p.window);
    if (wq_end > wq_begin) {  // tiles whose rows [t BQ + rg0, t BQ + rg0 + BQW) meet [wq_begin, wq_end)
      const int y = wq_begin - rg0 - BQW + 1;
      wt_begin = max(t_begin, y <= 0 ? 0 : (y + BQ - 1) / BQ);
      const int z = wq_end - rg0;
      wt_end = min(t_end, z <= 0 ? 0 : (z + BQ - 1) / BQ);
      if (wt_end < wt_begin) wt_end = wt_begin;
    }
  }
  // Tiles [t_full0, t_full1) need no mask for this wave: every row < Sq of its part sees all of its 32 * KPW keys.
  int t_full0 = t_begin, t_full1 = t_end;
  if constexpr (MASK) {
    if (p.causal) {
      const int a = kw0 + 32 * KPW - 1 - p.offset - rg0;  // first row that sees the wave's last key, less rg0
      t_full0 = a <= 0 ? t_begin : min(t_end, max(t_begin, (a + BQ - 1) / BQ));
    }
    if (p.window > 0) {
      const int last = kw0 + p.window - p.offset - 1;  // last query row that sees the wave's first key
      const int v = last + 1 - rg0 - BQW + BQ;          // tiles t < v / BQ end their group rows by last
      t_full1 = v <= 0 ? t_full0 : min(t_end, v / BQ);
    }
  }
  if (t_full1 * BQ > p.Sq) t_full1 = p.Sq / BQ;  // ragged last tile
  if (EPI == kColKF && !p.er_lane32) t_full1 = t_full0;  // exp_rand offsets too wide for the full-tile loads
  if (EPI == kColAnyGe && !p.thr_lane32) t_full1 = t_full0;  // threshold offsets too wide for the full-tile loads
  if (t_full1 < t_full0) t_full1 = t_full0;

  // Direct-load lane constants (as the forward's K tiles).
  const int rr = lane >> 4;
  const uint32_t src_chunk = (uint32_t)((lane & 15) ^ (rr << 2));
  uint32_t q_voff = (uint32_t)(rr * q_ss_b) + src_chunk * 16u;
  asm volatile("" : "+v"(q_voff));
  const uint32_t smem_base = (uint32_t)(size_t)((lds_char*)smem);

  auto issue = [&](int t) {
    const uint32_t stage = smem_base + (uint32_t)((t % NSTAGE) * STAGE_B);
    const uint32_t qdst = stage + (uint32_t)(GPW * w * GROUP_B);
    const int row0 = t * BQ + 4 * GPW * w;
    if ((t + 1) * BQ <= p.Sq) {
      const char* qb = qp + (int64_t)row0 * q_ss_b;
#pragma unroll
      for (int j = 0; j < GPW; ++j) dma16(qdst + j * GROUP_B, qb + 4 * j * q_ss_b, q_voff);
    } else {  // ragged last tile: rows past the end re-read the last row (masked)
#pragma unroll
      for (int j = 0; j < GPW; ++j) {
        const int64_t row = min(row0 + 4 * j + rr, p.Sq - 1);
        dma16(qdst + j * GROUP_B, qp + row * q_ss_b + src_chunk * 16);
      }
    }
    if (w == NW - 1) {
#pragma unroll
      for (int i = 0; i < NLSE; ++i) dma4(stage + QT_B + 256 * i, lsep + min(t * BQ + 64 * i + lane, p.Sq - 1));
    }
  };

  // Q fragment (row 32mb + r, chunk 2kk + g) addressing, as the forward's K fragments.
  const int s4 = r & 3;
  const uint32_t q_lane = (uint32_t)((rg0 / 4 + (r >> 2)) * GROUP_B + s4 * ROW_B + 16 * g);
  uint32_t xq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xq[i] = q_lane + 64u * (uint32_t)(i ^ s4);

  constexpr bool PK = REFROUND && !SOFTCAP && std::is_same<T, F16>::value;
  const float c = PK ? kLog2e : score_coeff<SOFTCAP, REFROUND>(p);
  const float cy = EPI == kColKF ? c * p.kf_inv_tau : 0.f;  // KeyFormer: score -> exp2 domain / tau
  ColAcc<EPI> acc[KPW];
  const int kjc = min(kj, p.Sk - 1);
  const float* erp = EPI == kColKF ? p.er + b * p.er_sb + h * p.er_sh : nullptr;  // KeyFormer exp_rand of (b, h)
  // KeyFormer exp_rand of (row, kjc) for tiles whose rows all exist: a wave-uniform tile address (scalar registers)
  // plus a 32-bit offset, this lane's part (rows 4g apart, column kjc) plus the row's, one add per load.
  const uint32_t er_lane_b = EPI == kColKF ? (uint32_t)((4 * g * p.er_ss + kjc) * 4) : 0u;
  // Corm's thresholds of (row, kjc), addressed the same way.
  const uint32_t thr_lane_b = EPI == kColAnyGe ? (uint32_t)((4 * g * p.thr_rs + kjc) * 4) : 0u;

  // S = Q . K^T of query tile t (its LDS stage) into s.
  auto qk_t = [&](const int t, f32x16 (&s)[NSB]) __attribute__((always_inline)) {
    const uint32_t st = smem_base + (uint32_t)((t % NSTAGE) * STAGE_B);
    uint32_t qb[4];  // opaque per-stage bases (reads at base + immediate offset)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qb[i] = st + xq[i];
      if constexpr (NSTAGE == 3) asm volatile("" : "+v"(qb[i]));
    }
#pragma unroll
    for (int i = 0; i < NSB; ++i) s[i] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const V8 a = lds_read<V8>(qb[kk >> 1] + mb * 8 * GROUP_B + 32 * (kk & 1));
#pragma unroll
        for (int kb = 0; kb < KPW; ++kb) s[kb * NMB + mb] = mfma32(a, kf[kb][kk], s[kb * NMB + mb]);
      }
    }
  };
  auto epi_t = [&](const int t, const f32x16 (&sacc)[NSB], const float (&ev)[NMB][16], const float (&tv)[NMB][16],
                   auto masked) __attribute__((always_inline)) {
    uint32_t lb = smem_base + (uint32_t)((t % NSTAGE) * STAGE_B) + QT_B + 4 * rg0 + 16 * g;  // this lane's lse
    if constexpr (NSTAGE == 3) asm volatile("" : "+v"(lb));
    // Visibility of (row o of the tile, this lane's key): causal rel >= 0, window rel < window, row < Sq.
    const int rows_left = p.Sq - t * BQ - rg0 - 4 * g;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      f32x4 lv[4];
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) lv[jq] = lds_read<f32x4>(lb + 4 * (32 * mb + 8 * jq));
#pragma unroll
      for (int kb = 0; kb < KPW; ++kb) {
      const f32x16& sb = sacc[kb * NMB + mb];
      const int rel0 = t * BQ + rg0 + 4 * g + p.offset - (kj + 32 * kb);
      f16x2 hs[8];
      if constexpr (PK) {
#pragma unroll
        for (int jp = 0; jp < 8; ++jp) hs[jp] = ref_scores_f16(sb[2 * jp], sb[2 * jp + 1], p);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float x;
        if constexpr (PK) x = (float)hs[j >> 1][j & 1];
        else x = score_value<T, SOFTCAP, REFROUND>(sb[j], p);
        const float l2 = LSE2 ? lv[j >> 2][j & 3] : lv[j >> 2][j & 3] * kLog2e;
        const int o = 32 * mb + 8 * (j >> 2) + (j & 3);
        float pe;
        if constexpr (EPI == kColKF)  // kf_prob with x * c folded into one fma against c / tau
          pe = __builtin_amdgcn_exp2f(fmaf(x, cy, -fmaf(__builtin_amdgcn_logf(ev[mb][j]), p.kf_inv_tau, l2)));
        else
          pe = fast_exp2(fmaf(x, c, -l2));
        bool valid = true, vis = true;
        if constexpr (decltype(masked)::value) {
          valid = o < rows_left;
          bool ok = valid;
          if constexpr (MASK) {
            if (p.causal) ok = ok && rel0 + o >= 0;
            if (p.window > 0) ok = ok && rel0 + o < p.window;
          }
          pe = ok ? pe : 0.f;
          vis = ok;
        }
        // Corm compares visible pairs here; the masked ones (p = 0) are ORed in by corm_masked_or_kernel
        if constexpr (EPI == kColAnyGe) acc[0].any |= vis && pe >= tv[mb][j];
        else acc[kb].add(pe, valid, min(t * BQ + rg0 + 4 * g + o, p.Sq - 1), min(kjc + 32 * kb, p.Sk - 1), p);
      }
      }
    }
  };

  auto tile = [&](const int t, auto masked) {
    float ev[NMB][16];
    if constexpr (EPI == kColKF) {
      if constexpr (!decltype(masked)::value) {  // every row of the tile exists (and er_lane32 holds)
        const char* rb = reinterpret_cast<const char*>(erp + (int64_t)(t * BQ) * p.er_ss);
        uint32_t ss_b = (uint32_t)(p.er_ss * 4);
        asm volatile("" : "+s"(ss_b));  // per tile: keeps the 64 offsets from being hoisted into registers
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const uint32_t row_b = (uint32_t)(32 * mb + 8 * (j >> 2) + (j & 3)) * ss_b;
            ev[mb][j] = *reinterpret_cast<const float*>(rb + (er_lane_b + row_b));
          }
      } else {  // rows past the end read the last row (their p is masked)
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int j = 0; j < 16; ++j)
            ev[mb][j] = erp[(int64_t)min(t * BQ + 4 * g + 32 * mb + 8 * (j >> 2) + (j & 3), p.Sq - 1) * p.er_ss + kjc];
      }
    }
    // Corm: the tile's thresholds for this lane's key, requested before the QK^T MFMAs so that the loads overlap
    // them (corm.py:35-37 compares each p with thr[i][j])
    float tv[NMB][16];
    if constexpr (EPI == kColAnyGe) {
      if constexpr (!decltype(masked)::value) {  // every row of the tile exists (and thr_lane32 holds)
        const char* rb = reinterpret_cast<const char*>(p.thr + (int64_t)(t * BQ) * p.thr_rs);
        uint32_t ss_b = (uint32_t)(p.thr_rs * 4);
        asm volatile("" : "+s"(ss_b));  // per tile: keeps the 64 offsets from being hoisted into registers
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const uint32_t row_b = (uint32_t)(32 * mb + 8 * (j >> 2) + (j & 3)) * ss_b;
            tv[mb][j] = *reinterpret_cast<const float*>(rb + (thr_lane_b + row_b));
          }
      } else {  // rows past the end read the last row (they take no part)
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int j = 0; j < 16; ++j)
            tv[mb][j] = p.thr[(int64_t)min(t * BQ + 4 * g + 32 * mb + 8 * (j >> 2) + (j & 3), p.Sq - 1) * p.thr_rs + kjc];
      }
    }
    f32x16 sacc[NSB];
    qk_t(t, sacc);
    epi_t(t, sacc, ev, tv, masked);
  };

#pragma unroll
  for (int i = 0; i < NSTAGE - 1; ++i)
    if (t_begin + i < t_end) issue(t_begin + i);
  // Corm: whether this wave's keys are all decided (no tile of its range left, or every key flagged).
  bool wave_done = wt_begin >= wt_end;
  // One pipelined step: the mask-free epilogue of tile t (scores in sc) and S of tile t+1 (into sn), in a fixed
  // order of 32 fenced steps, one per MFMA. Step i runs the QK^T MFMA of Q fragment f = i / KPW (k-step f / NMB,
  // query block f % NMB) with key block i % KPW, reads a later fragment when it starts a fragment, and takes the
  // exponentials and sums of score pair q = i / KPW (pair q % 8 of query block q / 8) of that key block; the lse
  // values of the next four rows are read when a group of two pairs starts. (Left to the compiler, the fragment
  // reads move to the front and the form spills.)
  auto pipe_step = [&](const int t, const f32x16 (&sc)[NSB], f32x16 (&sn)[NSB]) __attribute__((always_inline)) {
    static_assert(NSB == 4, "32 steps: 8 k-steps x 4 score blocks, 4 score blocks x 8 score pairs");
    constexpr int NF = 32 / KPW;       // Q fragments of a tile
    constexpr int NLG = 16 / KPW;      // groups of two score pairs (four rows' lse values) per key block
    const uint32_t stc = smem_base + (uint32_t)((t % NSTAGE) * STAGE_B);
    const uint32_t stn = smem_base + (uint32_t)(((t + 1) % NSTAGE) * STAGE_B);
    // per-stage base registers, opaque to the compiler, so that every read is base + immediate offset
    uint32_t qb[4], lb = stc + QT_B + 4 * rg0 + 16 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qb[i] = stn + xq[i];
      asm volatile("" : "+v"(qb[i]));
    }
    asm volatile("" : "+v"(lb));
    auto qread = [&](const int f) __attribute__((always_inline)) {
      const int kk = f / NMB, mb = f % NMB;
      return lds_read<V8>(qb[kk >> 1] + mb * 8 * GROUP_B + 32 * (kk & 1));
    };
    auto lread = [&](const int lg) __attribute__((always_inline)) {  // lse of the rows of pairs 2lg, 2lg+1
      return lds_read<f32x4>(lb + 4 * (32 * (lg >> 2) + 8 * (lg & 3)));
    };
#pragma unroll
    for (int i = 0; i < NSB; ++i) sn[i] = f32x16{};
    // Q fragment ring of NA slots: fragment f + NA - 1 is read when fragment f starts, two steps before its first
    // MFMA either way (one key block: three slots, two fragments ahead; two key blocks: two slots, one fragment
    // ahead, each fragment feeding two steps)
    constexpr int NA = KPW == 2 ? 2 : 3;
    V8 a[NA];
    f32x4 lvb[2];
#pragma unroll
    for (int j = 0; j < NA - 1; ++j) a[j] = qread(j);
    lvb[0] = lread(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int f = i / KPW, kb = i % KPW;
      if (kb == 0 && f + NA - 1 < NF) a[(f + NA - 1) % NA] = qread(f + NA - 1);
      const int q = i / KPW, lg = q >> 1;
      if (i % (2 * KPW) == 0 && lg + 1 < NLG) lvb[(lg + 1) & 1] = lread(lg + 1);
      sn[kb * NMB + f % NMB] = mfma32(a[f % NA], kf[kb][f / NMB], sn[kb * NMB + f % NMB]);
      const int mb = q >> 3, jp = q & 7;
      const f32x16& sp = sc[kb * NMB + mb];
      const f32x4& lv = lvb[lg & 1];
      float x[2];
      if constexpr (PK) {
        const f16x2 hs = ref_scores_f16(sp[2 * jp], sp[2 * jp + 1], p);
        x[0] = (float)hs[0];
        x[1] = (float)hs[1];
      } else {
        x[0] = score_value<T, SOFTCAP, REFROUND>(sp[2 * jp], p);
        x[1] = score_value<T, SOFTCAP, REFROUND>(sp[2 * jp + 1], p);
      }
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float l2 = LSE2 ? lv[2 * (jp & 1) + e] : lv[2 * (jp & 1) + e] * kLog2e;
        acc[kb].add(fast_exp2(fmaf(x[e], c, -l2)), true, 0, kjc, p);
      }
#pragma unroll
      for (int k2 = 0; k2 < KPW; ++k2) acc[k2].pin();
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // PIPE: the mask-free tiles of a wave run software-pipelined, the QK^T MFMAs of tile t+1 in the same basic block
  // as the exponentials and sums of tile t (which are VALU work the MFMA pipe would otherwise wait out). Tile t+1
  // must then be in the LDS at the barrier of tile t, so every barrier waits for all copies issued before it, and
  // a third stage keeps tile t (its lse values) while tile t+2 lands.
  constexpr bool PIPE = NSTAGE == 3;
  static_assert(!PIPE || EPI == kColSum || EPI == kColSumSq, "three stages only for the pipelined epilogues");
  // Waits for the copies of tile t (PIPE: and of tile t+1), then the barrier after which tile t+NSTAGE-1 is
  // requested into the stage of tile t-1 (every wave has finished with it).
  auto sync = [&](const int t) -> bool {
    // Tiles t+1 .. t+after may stay in flight; the last wave issues NLSE more copies per tile.
    const int after = PIPE ? 0 : min(NSTAGE - 2, t_end - 1 - t);
    if (w == NW - 1) {
      if (NSTAGE >= 4 && after >= 2) wait_vmem<2 * (GPW + NLSE)>();
      else if (NSTAGE >= 3 && after >= 1) wait_vmem<GPW + NLSE>();
      else wait_vmem<0>();
    } else {
      if (NSTAGE >= 4 && after >= 2) wait_vmem<2 * GPW>();
      else if (NSTAGE >= 3 && after >= 1) wait_vmem<GPW>();
      else wait_vmem<0>();
    }
    if constexpr (EPI == kColAnyGe) {
      // Corm ORs over the query rows: once every key of every wave is flagged, no later tile can change the
      // result, and the workgroup stops. The vote doubles as the tile's barrier; the copies of this tile have
      // landed and none is in flight yet (NSTAGE 2), so nothing still writes into the LDS when it stops.
      static_assert(EPI != kColAnyGe || NSTAGE == 2, "the early stop assumes no copy in flight at the barrier");
      if (__syncthreads_and(wave_done)) return false;
    } else {
      __syncthreads();
    }
    if (t + NSTAGE - 1 < t_end) issue(t + NSTAGE - 1);
    return true;
  };
  auto step = [&](const int t, auto masked) -> bool {
    if (!sync(t)) return false;
    if (t >= wt_begin && t < wt_end) {
      tile(t, masked);
      if constexpr (EPI == kColAnyGe) {
        // this lane's key is decided when either half of its rows flagged it (keys past the end count as decided)
        const bool decided = (acc[0].any | __shfl_xor(acc[0].any, 32, 64)) != 0 || kj >= p.Sk;
        wave_done = t + 1 >= wt_end || __all(decided);
      }
    }
    return true;
  };
  bool go = true;
  for (int t = t_begin; go && t < t_full0; ++t) go = step(t, std::true_type{});
  // The mask-free range lies inside the wave's range whenever the wave has keys (kw0 < Sk).
  if (PIPE && t_full1 - t_full0 >= 2 && t_full0 >= wt_begin && t_full1 <= wt_end) {
    // scores of two tiles in flight, in two buffers that swap roles every step (loop unrolled by two)
    f32x16 sa[NSB], sb[NSB];
    float none[NMB][16];  // KeyFormer / Corm inputs, never read by these epilogues
    int t = t_full0;
    sync(t);
    qk_t(t, sa);
    pipe_step(t, sa, sb);
    for (++t;;) {
      sync(t);
      if (t + 1 >= t_full1) {
        epi_t(t, sb, none, none, std::false_type{});
        break;
      }
      pipe_step(t, sb, sa);
      sync(++t);
      if (t + 1 >= t_full1) {
        epi_t(t, sa, none, none, std::false_type{});
        break;
      }
      pipe_step(t, sa, sb);
      ++t;
    }
  } else {
    for (int t = t_full0; go && t < t_full1; ++t) go = step(t, std::false_type{});
  }
  for (int t = t_full1; go && t < t_end; ++t) go = step(t, std::true_type{});

  if constexpr (NG == 1) {
    acc[0].store(p, bh, kj, g);
  } else {
    // Row group 1 leaves its sums (lane halves added) in the LDS; group 0 adds them to its own and stores.
    wait_vmem<0>();
    __syncthreads();  // every wave is done with the Q stages
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int kb = 0; kb < KPW; ++kb) {
      acc[kb].s += __shfl_xor(acc[kb].s, 32, 64);
      if constexpr (EPI == kColSumSq) acc[kb].s2 += __shfl_xor(acc[kb].s2, 32, 64);
      const int key = 32 * (KPW * wi + kb) + r;  // key within the workgroup
      if (gw == 1 && g == 0) {
        red[key] = acc[kb].s;
        if constexpr (EPI == kColSumSq) red[BK + key] = acc[kb].s2;
      }
    }
    __syncthreads();
    if (gw == 0 && g == 0) {
#pragma unroll
      for (int kb = 0; kb < KPW; ++kb) {
        const int key = 32 * (KPW * wi + kb) + r, kjb = kj + 32 * kb;
        if (kjb < p.Sk) {
          p.colsum[(int64_t)bh * p.Sk + kjb] = acc[kb].s + red[key];
          if constexpr (EPI == kColSumSq) p.colsum2[(int64_t)bh * p.Sk + kjb] = acc[kb].s2 + red[BK + key];
        }
      }
    }
  }
}

template <typename T, int D, int BN, bool MASK, bool SOFTCAP, int REFROUND>
void launch_fwd(const AttnParams& p, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  hipLaunchKernelGGL((attn_fwd_kernel<T, D, BN, MASK, SOFTCAP, REFROUND>), dim3(grid), dim3(kThreads), 0, st, p);
}

template <typename T, int D, bool MASK, bool SOFTCAP, int REFROUND, int EPI>
void launch_colsum(const AttnParams& p, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  hipLaunchKernelGGL((attn_colsum_kernel<T, D, MASK, SOFTCAP, REFROUND, EPI>), dim3(grid), dim3(kThreads), 0, st, p);
}

// head_dim 128 configuration (measured on MI355X, config 2): 8 waves x 32 rows, 128-key tiles, 2-stage ring.
#ifndef DGG_D128_NW
#define DGG_D128_NW 8
#endif
#ifndef DGG_D128_BN
#define DGG_D128_BN 128
#endif
// DGG_D128_OCC: waves per SIMD the register budget is sized for (2; 3 with DGG_D128_NW=4 DGG_D128_BN=32 is the
// three-waves-per-SIMD form, whose LDS fits three workgroups per CU only at 32-key tiles).
#ifndef DGG_D128_OCC
#define DGG_D128_OCC 2
#endif
constexpr int kD128NQB = 1, kD128NW = DGG_D128_NW, kD128BN = DGG_D128_BN, kD128NS = 2;
constexpr int kD128BM = 32 * kD128NQB * kD128NW;  // query rows per workgroup (head_dim 128)

template <typename T, bool MASK, bool SOFTCAP, int REFROUND>
void launch_fwd_d128(const AttnParams& p, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  if (!REFROUND && p.lse == nullptr)
    hipLaunchKernelGGL(
        (attn_fwd_dma_kernel<T, 128, kD128NQB, kD128NW, kD128BN, kD128NS, DGG_D128_OCC, MASK, SOFTCAP, REFROUND, !REFROUND>),
        dim3(grid), dim3(64 * kD128NW), 0, st, p);
  else
    hipLaunchKernelGGL(
        (attn_fwd_dma_kernel<T, 128, kD128NQB, kD128NW, kD128BN, kD128NS, DGG_D128_OCC, MASK, SOFTCAP, REFROUND, false>),
        dim3(grid), dim3(64 * kD128NW), 0, st, p);
}

// head_dim 256 configuration: 4 waves x 32 rows (one wave per SIMD), DGG_D256_BN-key tiles, 2-stage ring.
#ifndef DGG_D256_BN
#define DGG_D256_BN 64
#endif
constexpr int kD256NW = 4, kD256BN = DGG_D256_BN, kD256NS = 2;
constexpr int kD256BM = 32 * kD256NW;

// DGG_D256_PIPE (default 1): the software-pipelined kernel of attention_d256.hip for the scores in fp32; 0 keeps
// every head_dim-256 launch on attn_fwd_dma_kernel (for A/B measurements).
#ifndef DGG_D256_PIPE
#define DGG_D256_PIPE 1
#endif

template <typename T, bool MASK, bool SOFTCAP, int REFROUND>
void launch_fwd_d256(const AttnParams& p, hipStream_t st) {
  if (DGG_D256_PIPE && !REFROUND) return launch_attn_d256_pipe(p, std::is_same<T, BF16>::value, st);
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  if (!REFROUND && p.lse == nullptr)
    hipLaunchKernelGGL((attn_fwd_dma_kernel<T, 256, 1, kD256NW, kD256BN, kD256NS, 1, MASK, SOFTCAP, REFROUND, !REFROUND>),
                       dim3(grid), dim3(64 * kD256NW), 0, st, p);
  else
    hipLaunchKernelGGL((attn_fwd_dma_kernel<T, 256, 1, kD256NW, kD256BN, kD256NS, 1, MASK, SOFTCAP, REFROUND, false>),
                       dim3(grid), dim3(64 * kD256NW), 0, st, p);
}

// Reference-rounding mode of a launch (the REFROUND template argument): 0 off, 1 the scores rounded as the
// reference rounds them (score_value).
template <int D, bool SOFTCAP, typename F>
void with_ref_mode(bool ref, const AttnParams& p, F&& f) {
  if (ref) f(std::integral_constant<int, 1>{});
  else f(std::integral_constant<int, 0>{});
}

template <typename T, int D, bool MASK, bool SOFTCAP>
void pick_fwd_ref(const AttnParams& p, bool ref, hipStream_t st) {
  constexpr int BN = D >= 256 ? 32 : 64;
  with_ref_mode<D, SOFTCAP>(ref, p, [&](auto mode) {
    constexpr int R = decltype(mode)::value;
    if constexpr (D == 128) launch_fwd_d128<T, MASK, SOFTCAP, R>(p, st);
    else if constexpr (D == 256) launch_fwd_d256<T, MASK, SOFTCAP, R>(p, st);
    else launch_fwd<T, D, BN, MASK, SOFTCAP, R>(p, st);
  });
}
template <typename T, int D>
void pick_fwd(const AttnParams& p, bool ref, hipStream_t st) {
  const bool mask = p.causal || p.window > 0;
  const bool sc = p.softcap > 0.f;
  if (mask) {
    if (sc) pick_fwd_ref<T, D, true, true>(p, ref, st);
    else pick_fwd_ref<T, D, true, false>(p, ref, st);
  } else {
    if (sc) pick_fwd_ref<T, D, false, true>(p, ref, st);
    else pick_fwd_ref<T, D, false, false>(p, ref, st);
  }
}
// head_dim 128 column sums (measured on MI355X, config 4): 8 waves x 32 keys, 128-row query tiles, 2 stages.
// DGG_COL_PIPE (default 1): the sum epilogues (H2O / SnapKV, RoCo) run the software-pipelined 3-stage form.
#ifndef DGG_COL_PIPE
#define DGG_COL_PIPE 1
#endif
// DGG_COL_KPW: 32-key blocks per wave in the pipelined form (2; 1: 8 waves x 32 keys over 128-row tiles).
#ifndef DGG_COL_KPW
#define DGG_COL_KPW 2
#endif
constexpr int kC128NW = 8, kC128BQ = 128, kC128NS = 2;
constexpr int kC128BK = 32 * kC128NW;  // keys per workgroup (head_dim 128)

template <typename T, bool MASK, bool SOFTCAP, int REFROUND, int EPI>
void launch_colsum_d128(const AttnParams& p, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  // (the reference-rounded soft-cap's score chain is too long for a fixed-order step: it keeps the plain form)
  constexpr bool PIPE = DGG_COL_PIPE && (EPI == kColSum || EPI == kColSumSq) && !(SOFTCAP && REFROUND);
  constexpr int NS = PIPE ? 3 : kC128NS;
  // The pipelined form: 64 keys per wave, the 8 waves in two row groups of 4 (each group takes 64 rows of every
  // 128-row query tile); the same 256 keys per workgroup.
  constexpr int KPW = PIPE ? DGG_COL_KPW : 1;
  constexpr int NW = kC128NW, BQ = kC128BQ;
  static_assert(32 * NW == kC128BK, "keys per workgroup");
  if (p.lse_base2)
    hipLaunchKernelGGL((attn_colsum_d128_kernel<T, NW, KPW, BQ, NS, MASK, SOFTCAP, REFROUND, true, EPI>),
                       dim3(grid), dim3(64 * NW), 0, st, p);
  else
    hipLaunchKernelGGL((attn_colsum_d128_kernel<T, NW, KPW, BQ, NS, MASK, SOFTCAP, REFROUND, false, EPI>),
                       dim3(grid), dim3(64 * NW), 0, st, p);
}

template <typename T, int D, bool MASK, bool SOFTCAP, int REFROUND, int EPI>
void launch_col(const AttnParams& p, hipStream_t st) {
  if constexpr (D == 128) launch_colsum_d128<T, MASK, SOFTCAP, REFROUND, EPI>(p, st);
  else launch_colsum<T, D, MASK, SOFTCAP, REFROUND, EPI>(p, st);
}
template <typename T, int D, bool MASK, bool SOFTCAP>
void pick_col_ref(const AttnParams& p, bool ref, hipStream_t st) {
  with_ref_mode<D, SOFTCAP>(ref, p, [&](auto mode) {
    launch_col<T, D, MASK, SOFTCAP, decltype(mode)::value, kColSum>(p, st);
  });
}
// The RoCo / Corm epilogues exist for the mask-checking, soft-cap-free variants only (the reference cases are
// causal and have no soft-cap); the host rejects a soft-cap with them.
template <typename T, int D, int EPI>
void pick_col_epi(const AttnParams& p, bool ref, hipStream_t st) {
  with_ref_mode<D, false>(ref, p, [&](auto mode) { launch_col<T, D, true, false, decltype(mode)::value, EPI>(p, st); });
}
template <typename T, int D>
void pick_col(const AttnParams& p, bool ref, int epi, hipStream_t st) {
  if (epi == kColSumSq) return pick_col_epi<T, D, kColSumSq>(p, ref, st);
  if (epi == kColAnyGe) return pick_col_epi<T, D, kColAnyGe>(p, ref, st);
  if (epi == kColKF) return pick_col_epi<T, D, kColKF>(p, ref, st);
  const bool mask = p.causal || p.window > 0;
  const bool sc = p.softcap > 0.f;
  if (mask) {
    if (sc) pick_col_ref<T, D, true, true>(p, ref, st);
    else pick_col_ref<T, D, true, false>(p, ref, st);
  } else {
    if (sc) pick_col_ref<T, D, false, true>(p, ref, st);
    else pick_col_ref<T, D, false, false>(p, ref, st);
  }
}

template <typename T, int D, bool MASK, int REFROUND>
void launch_kf_rowlse(const AttnParams& p, bool vec, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  if (vec) hipLaunchKernelGGL((attn_kf_rowlse_kernel<T, D, MASK, REFROUND, true>), dim3(grid), dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((attn_kf_rowlse_kernel<T, D, MASK, REFROUND, false>), dim3(grid), dim3(kThreads), 0, st, p);
}
template <typename T, int D>
void pick_kf_rowlse(const AttnParams& p, bool ref, bool vec, hipStream_t st) {
  const bool mask = p.causal || p.window > 0;
  with_ref_mode<D, false>(ref, p, [&](auto mode) {
    constexpr int R = decltype(mode)::value;
    if (mask) launch_kf_rowlse<T, D, true, R>(p, vec, st);
    else launch_kf_rowlse<T, D, false, R>(p, vec, st);
  });
}

}  // namespace

namespace dgg_attn {

// Shared host-side validation of the attention arguments.
int validate_attn(const char* op, const void* q, const void* k, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq,
                  int64_t Hkv, int64_t D, const int64_t* strides, int nstrides, float scale, float softcap,
                  int64_t window, int dtype) {
  DGG_REQUIRE(dtype == DGG_F16 || dtype == DGG_BF16 || dtype == DGG_F32, DGG_ERR_DTYPE,
              "%s: dtype code %d not supported (attention kernels take f32, f16 or bf16)", op, dtype);
  DGG_REQUIRE(D == 64 || D == 128 || D == 256, DGG_ERR_UNSUPPORTED, "%s: head_dim %lld not supported (64, 128, 256)",
              op, (long long)D);
  DGG_REQUIRE(B >= 0 && Sq >= 0 && Sk >= 0, DGG_ERR_SHAPE, "%s: negative size", op);
  DGG_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0, DGG_ERR_SHAPE,
              "%s: query heads (%lld) must be a positive multiple of kv heads (%lld)", op, (long long)Hq,
              (long long)Hkv);
  DGG_REQUIRE(Sq < (1ll << 30) && Sk < (1ll << 30) && B < (1ll << 20) && Hq < (1ll << 16), DGG_ERR_SHAPE,
              "%s: size too large", op);
  DGG_REQUIRE(B * Hq * ((std::max(Sq, Sk) + 127) / 128) < (1ll << 31), DGG_ERR_SHAPE, "%s: grid too large", op);
  DGG_REQUIRE(strides != nullptr, DGG_ERR_NULL, "%s: strides is NULL", op);
  for (int i = 0; i < nstrides; ++i) {
    DGG_REQUIRE(strides[i] >= 0 && strides[i] % 8 == 0, DGG_ERR_STRIDE,
                "%s: stride[%d] = %lld must be a non-negative multiple of 8 elements", op, i, (long long)strides[i]);
    // in-tile row offsets are 32-bit: 256 rows of the sequence stride must stay below 2^31 elements
    DGG_REQUIRE(i % 3 != 1 || strides[i] < (1ll << 23), DGG_ERR_STRIDE,
                "%s: sequence stride[%d] = %lld must be < 2^23 elements", op, i, (long long)strides[i]);
  }
  DGG_REQUIRE(std::isfinite(scale) && scale > 0.f, DGG_ERR_SHAPE, "%s: scale must be finite and > 0", op);
  DGG_REQUIRE(softcap >= 0.f && std::isfinite(softcap), DGG_ERR_SHAPE, "%s: softcap must be >= 0 (0 = off)", op);
  DGG_REQUIRE(window >= 0 && window < (1ll << 30), DGG_ERR_SHAPE, "%s: window must be >= 0 (0 = off)", op);
  // q is read whenever there are query rows (the forward kernels load it even when Sk == 0), k whenever there are
  // keys.
  if (B > 0 && Sq > 0) {
    DGG_REQUIRE(q != nullptr, DGG_ERR_NULL, "%s: null q pointer", op);
    DGG_REQUIRE(dgg::aligned16(q), DGG_ERR_ALIGN, "%s: q must be 16-byte aligned", op);
  }
  if (B > 0 && Sk > 0) {
    DGG_REQUIRE(k != nullptr, DGG_ERR_NULL, "%s: null k pointer", op);
    DGG_REQUIRE(dgg::aligned16(k), DGG_ERR_ALIGN, "%s: k must be 16-byte aligned", op);
  }
  return DGG_OK;
}

AttnParams make_params(const void* q, const void* k, const void* v, void* o, int64_t B, int64_t Sq, int64_t Sk,
                       int64_t Hq, int64_t Hkv, int64_t D, float scale, float softcap, int64_t window, uint32_t flags) {
  AttnParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.B = (int)B;
  p.Sq = (int)Sq;
  p.Sk = (int)Sk;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.group = (int)(Hq / Hkv);
  p.causal = (flags & DGG_ATTN_CAUSAL) ? 1 : 0;
  p.lse_base2 = (flags & DGG_ATTN_LSE_BASE2) ? 1 : 0;
  p.window = (int)window;
  p.offset = (int)(Sk - Sq);
  p.scale = scale;
  // The reference divides its scores by math.sqrt(D) (attn.py:29); torch takes that Python float to fp32 and
  // multiplies by the fp32 reciprocal. A scale other than the default is taken as 1 / divisor.
  const double root = std::sqrt((double)D);
  p.ref_div = scale == (float)(1.0 / root) ? (float)root : (float)(1.0 / (double)scale);
  p.ref_rcp = 1.0f / p.ref_div;
  p.c_fast = scale * kLog2e;
  p.softcap = softcap;
  p.inv_softcap = softcap > 0.f ? 1.0f / softcap : 0.f;
  p.sc_a = softcap > 0.f ? 2.0f * scale / softcap * kLog2e : 0.f;
  p.sc_b = softcap * kLog2e;
  return p;
}

}  // namespace dgg_attn

namespace {
// Shared body of dgg_attn_prefill and dgg_attn_prefill_rope (rope: rotate the query rows by the table rope_cs).
int prefill_impl(const char* op, const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                 int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides, float scale,
                 float softcap, int64_t window, uint32_t flags, int dtype, bool rope, const float* rope_cs,
                 void* stream) {
  if (int rc = validate_attn(op, q, k, B, Sq, Sk, Hq, Hkv, D, strides, 12, scale, softcap, window, dtype)) return rc;
  if (rope)
    DGG_REQUIRE(D == 128 && dtype != DGG_F32, DGG_ERR_UNSUPPORTED,
                "%s: the fused rotary takes head_dim 128 (pos_encoding.cu:195) and 16-bit inputs", op);
  if (B == 0 || Sq == 0) return DGG_OK;
  DGG_REQUIRE(o && (v || Sk == 0), DGG_ERR_NULL, "%s: null v/o pointer", op);
  DGG_REQUIRE(dgg::aligned16(v) && dgg::aligned16(o), DGG_ERR_ALIGN, "%s: v/o must be 16-byte aligned", op);
  if (rope) {
    DGG_REQUIRE(rope_cs != nullptr, DGG_ERR_NULL, "%s: null rotary table", op);
    DGG_REQUIRE(((uintptr_t)rope_cs & 31u) == 0, DGG_ERR_ALIGN, "%s: the rotary table must be 32-byte aligned", op);
  }
  AttnParams p = make_params(q, k, v, o, B, Sq, Sk, Hq, Hkv, D, scale, softcap, window, flags);
  p.rope_cs = rope_cs;
  p.lse = lse;
  p.q_sb = strides[0]; p.q_ss = strides[1]; p.q_sh = strides[2];
  p.k_sb = strides[3]; p.k_ss = strides[4]; p.k_sh = strides[5];
  p.v_sb = strides[6]; p.v_ss = strides[7]; p.v_sh = strides[8];
  p.o_sb = strides[9]; p.o_ss = strides[10]; p.o_sh = strides[11];
  const bool ref = (flags & DGG_ATTN_REF_ROUNDING) != 0;
  hipStream_t st = dgg::as_stream(stream);
  // Sk == 0 still launches and writes o = 0 (the reference's P.V over an empty key axis) and lse = -inf.
  if (dtype == DGG_F32) {  // fp32 has no 16-bit rounding point: reference rounding changes nothing
    p.n_tiles = (int)((Sq + f32_rows_per_tile() - 1) / f32_rows_per_tile());
    launch_attn_f32_fwd(p, (int)D, st);
    return dgg::check_launch(op);
  }
  const int64_t bm = D == 128 ? kD128BM : D == 256 ? kD256BM : kBM;
  p.n_tiles = (int)((Sq + bm - 1) / bm);
  if (dtype == DGG_BF16) {
    if (D == 64) pick_fwd<BF16, 64>(p, ref, st);
    else if (D == 128) pick_fwd<BF16, 128>(p, ref, st);
    else pick_fwd<BF16, 256>(p, ref, st);
  } else {
    if (D == 64) pick_fwd<F16, 64>(p, ref, st);
    else if (D == 128) pick_fwd<F16, 128>(p, ref, st);
    else pick_fwd<F16, 256>(p, ref, st);
  }
  return dgg::check_launch(op);
}
}  // namespace

extern "C" int dgg_attn_prefill(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                                int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides,
                                float scale, float softcap, int64_t window, uint32_t flags, int dtype, void* stream) {
  return prefill_impl("attn_prefill", q, k, v, o, lse, B, Sq, Sk, Hq, Hkv, D, strides, scale, softcap, window, flags,
                      dtype, false, nullptr, stream);
}

extern "C" int dgg_attn_prefill_rope(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                                     int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D,
                                     const int64_t* strides, float scale, float softcap, int64_t window,
                                     uint32_t flags, int dtype, const float* q_cos_sin, void* stream) {
  return prefill_impl("attn_prefill_rope", q, k, v, o, lse, B, Sq, Sk, Hq, Hkv, D, strides, scale, softcap, window,
                      flags, dtype, true, q_cos_sin, stream);
}

namespace {
// Corm over the masked pairs (corm.py:35-37 compares every query row, masked pairs included): a masked pair of a
// row that sees at least one key has p = 0 (softmax of -inf), so it flags its key when thr[i][j] <= 0; a row that
// sees no key at all has NaN probabilities (0 / 0) and flags nothing. The column kernels compare the visible pairs
// only; this kernel, run after them on the same stream, sets any_out[bh][j] = 1 for every (batch, head) when some
// masked pair of a non-empty row has thr[i][j] <= 0 (the thresholds are shared by all heads). One thread per key and
// chunk of kMaskedRows rows, reading only the masked part of the chunk: for causal the rows before the key's
// diagonal, for a window the rows past its end. Flags are written only when found, as plain byte stores of 1.
constexpr int kMaskedRows = 64;
__global__ void __launch_bounds__(256) corm_masked_or_kernel(const float* __restrict__ thr, int64_t rs, int Sq, int Sk,
                                                             int offset, int causal, int window, uint8_t* any_out,
                                                             int64_t nbh) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= Sk) return;
  const int r0 = blockIdx.y * kMaskedRows, r1 = min(Sq, r0 + kMaskedRows);
  // masked rows of key j: [a0, a1) before the diagonal (rows i + offset < j that see a key: i + offset >= 0),
  // [b0, r1) past the window (i + offset - j >= window)
  int a0 = r1, a1 = r1, b0 = r1;
  const int64_t diag = (int64_t)j - offset;  // first row that sees key j (causal)
  if (causal) {
    a0 = (int)max<int64_t>(r0, max<int64_t>(0, -(int64_t)offset));
    a1 = (int)min<int64_t>(r1, diag);
  }
  if (window > 0) b0 = (int)min<int64_t>(r1, max<int64_t>(r0, diag + window));  // never overlaps [a0, a1)
  bool hit = false;
#pragma unroll 8
  for (int i = a0; i < a1; ++i) hit |= thr[(int64_t)i * rs + j] <= 0.f;
#pragma unroll 8
  for (int i = b0; i < r1; ++i) hit |= thr[(int64_t)i * rs + j] <= 0.f;
  if (hit)
    for (int64_t bh = 0; bh < nbh; ++bh) any_out[bh * Sk + j] = 1;
}

// Shared body of dgg_attn_colsum and dgg_attn_colscore.
int colscore(const char* op, const void* q, const void* k, const float* lse, int epi, float* out0, float* out1,
             uint8_t* out_any, const float* thr, int64_t thr_row_stride, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq,
             int64_t Hkv, int64_t D, const int64_t* strides, float scale, float softcap, int64_t window, uint32_t flags,
             int dtype, void* stream) {
  if (int rc = validate_attn(op, q, k, B, Sq, Sk, Hq, Hkv, D, strides, 6, scale, softcap, window, dtype)) return rc;
  DGG_REQUIRE(epi == kColSum || epi == kColSumSq || epi == kColAnyGe, DGG_ERR_UNSUPPORTED, "%s: unknown epilogue %d", op,
              epi);
  DGG_REQUIRE(epi == kColSum || softcap == 0.f, DGG_ERR_UNSUPPORTED, "%s: epilogue %d takes no soft-cap", op, epi);
  if (B == 0 || Sk == 0) return DGG_OK;
  if (epi == kColAnyGe) {
    DGG_REQUIRE(out_any != nullptr, DGG_ERR_NULL, "%s: null output pointer", op);
    DGG_REQUIRE(Sq == 0 || thr != nullptr, DGG_ERR_NULL, "%s: null threshold pointer", op);
    DGG_REQUIRE(Sq == 0 || (thr_row_stride >= Sk && thr_row_stride < (1ll << 40)), DGG_ERR_STRIDE,
                "%s: threshold row stride %lld must be >= Sk (%lld)", op, (long long)thr_row_stride, (long long)Sk);
  } else {
    DGG_REQUIRE(out0 != nullptr && (epi != kColSumSq || out1 != nullptr), DGG_ERR_NULL, "%s: null output pointer", op);
  }
  DGG_REQUIRE(Sq == 0 || lse != nullptr, DGG_ERR_NULL, "%s: null lse pointer", op);
  AttnParams p = make_params(q, k, nullptr, nullptr, B, Sq, Sk, Hq, Hkv, D, scale, softcap, window, flags);
  p.lse = const_cast<float*>(lse);
  p.colsum = out0;
  p.colsum2 = out1;
  p.any_out = out_any;
  p.thr = thr;
  p.thr_rs = thr_row_stride;
  p.thr_lane32 = (132 * thr_row_stride + Sk) * 4 < (1ll << 31) ? 1 : 0;
  p.q_sb = strides[0]; p.q_ss = strides[1]; p.q_sh = strides[2];
  p.k_sb = strides[3]; p.k_ss = strides[4]; p.k_sh = strides[5];
  hipStream_t st = dgg::as_stream(stream);
  if (dtype == DGG_F32) {
    p.n_tiles = (int)((Sk + f32_rows_per_tile() - 1) / f32_rows_per_tile());
    launch_attn_f32_col(p, (int)D, epi, st);
  } else {
    const int64_t bk = D == 128 ? kC128BK : kCBK;
    p.n_tiles = (int)((Sk + bk - 1) / bk);
    const bool ref = (flags & DGG_ATTN_REF_ROUNDING) != 0;
    if (dtype == DGG_BF16) {
      if (D == 64) pick_col<BF16, 64>(p, ref, epi, st);
      else if (D == 128) pick_col<BF16, 128>(p, ref, epi, st);
      else pick_col<BF16, 256>(p, ref, epi, st);
    } else {
      if (D == 64) pick_col<F16, 64>(p, ref, epi, st);
      else if (D == 128) pick_col<F16, 128>(p, ref, epi, st);
      else pick_col<F16, 256>(p, ref, epi, st);
    }
  }
  if (epi == kColAnyGe && Sq > 0 && (p.causal || p.window > 0)) {
    const dim3 grid((unsigned)((Sk + 255) / 256), (unsigned)((Sq + kMaskedRows - 1) / kMaskedRows));
    hipLaunchKernelGGL(corm_masked_or_kernel, grid, dim3(256), 0, st, thr, thr_row_stride, (int)Sq, (int)Sk, p.offset,
                       p.causal, p.window, out_any, B * Hq);
  }
  return dgg::check_launch(op);
}
}  // namespace

namespace {
// exp_rand [B, Hq, Sq, Sk] fp32 with element strides er_strides = {batch, head, row} and unit key stride.
int validate_exp_rand(const char* op, const float* er, const int64_t* er_strides, int64_t Sq, float tau) {
  DGG_REQUIRE(er != nullptr && er_strides != nullptr, DGG_ERR_NULL, "%s: null exp_rand / strides", op);
  DGG_REQUIRE(((uintptr_t)er & 3u) == 0, DGG_ERR_ALIGN, "%s: exp_rand must be 4-byte aligned", op);
  for (int i = 0; i < 3; ++i)
    DGG_REQUIRE(er_strides[i] >= 0 && er_strides[i] < (1ll << 40), DGG_ERR_STRIDE, "%s: exp_rand stride[%d] invalid", op,
                i);
  DGG_REQUIRE(Sq <= 1 || er_strides[2] > 0, DGG_ERR_STRIDE, "%s: exp_rand row stride must be > 0", op);
  DGG_REQUIRE(std::isfinite(tau) && tau > 0.f, DGG_ERR_SHAPE, "%s: tau must be finite and > 0", op);
  return DGG_OK;
}
void set_exp_rand(AttnParams& p, const float* er, const int64_t* er_strides, float tau) {
  p.er = er;
  p.er_sb = er_strides[0];
  p.er_sh = er_strides[1];
  p.er_ss = er_strides[2];
  p.kf_inv_tau = 1.0f / tau;
  p.er_lane32 = (132 * er_strides[2] + p.Sk) * 4 < (1ll << 31) ? 1 : 0;
}
}  // namespace

extern "C" int dgg_attn_kf_rowlse(const void* q, const void* k, const float* exp_rand, const int64_t* er_strides,
                                  float* lse2, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D,
                                  const int64_t* strides, float scale, float tau, int64_t window, uint32_t flags,
                                  int dtype, void* stream) {
  const char* op = "attn_kf_rowlse";
  DGG_REQUIRE(dtype == DGG_F16 || dtype == DGG_BF16, DGG_ERR_DTYPE,
              "%s: dtype code %d not supported (the KeyFormer passes take f16 or bf16)", op, dtype);
  if (int rc = validate_attn(op, q, k, B, Sq, Sk, Hq, Hkv, D, strides, 6, scale, 0.f, window, dtype)) return rc;
  if (B == 0 || Sq == 0) return DGG_OK;
  DGG_REQUIRE(lse2 != nullptr, DGG_ERR_NULL, "%s: null lse output", op);
  DGG_REQUIRE(Sk > 0, DGG_ERR_SHAPE, "%s: Sk must be > 0", op);
  if (int rc = validate_exp_rand(op, exp_rand, er_strides, Sq, tau)) return rc;
  AttnParams p = make_params(q, k, nullptr, nullptr, B, Sq, Sk, Hq, Hkv, D, scale, 0.f, window, flags);
  p.lse = lse2;
  p.q_sb = strides[0]; p.q_ss = strides[1]; p.q_sh = strides[2];
  p.k_sb = strides[3]; p.k_ss = strides[4]; p.k_sh = strides[5];
  set_exp_rand(p, exp_rand, er_strides, tau);
  p.n_tiles = (int)((Sq + kBM - 1) / kBM);
  const bool vec = dgg::aligned16(exp_rand) && er_strides[0] % 4 == 0 && er_strides[1] % 4 == 0 && er_strides[2] % 4 == 0;
  const bool ref = (flags & DGG_ATTN_REF_ROUNDING) != 0;
  hipStream_t st = dgg::as_stream(stream);
  if (dtype == DGG_BF16) {
    if (D == 64) pick_kf_rowlse<BF16, 64>(p, ref, vec, st);
    else if (D == 128) pick_kf_rowlse<BF16, 128>(p, ref, vec, st);
    else pick_kf_rowlse<BF16, 256>(p, ref, vec, st);
  } else {
    if (D == 64) pick_kf_rowlse<F16, 64>(p, ref, vec, st);
    else if (D == 128) pick_kf_rowlse<F16, 128>(p, ref, vec, st);
    else pick_kf_rowlse<F16, 256>(p, ref, vec, st);
  }
  return dgg::check_launch(op);
}

extern "C" int dgg_attn_kf_colsum(const void* q, const void* k, const float* exp_rand, const int64_t* er_strides,
                                  const float* lse2, float* kf_score, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq,
                                  int64_t Hkv, int64_t D, const int64_t* strides, float scale, float tau,
                                  int64_t window, uint32_t flags, int dtype, void* stream) {
  const char* op = "attn_kf_colsum";
  DGG_REQUIRE(dtype == DGG_F16 || dtype == DGG_BF16, DGG_ERR_DTYPE,
              "%s: dtype code %d not supported (the KeyFormer passes take f16 or bf16)", op, dtype);
  if (int rc = validate_attn(op, q, k, B, Sq, Sk, Hq, Hkv, D, strides, 6, scale, 0.f, window, dtype)) return rc;
  if (B == 0 || Sk == 0) return DGG_OK;
  DGG_REQUIRE(kf_score != nullptr, DGG_ERR_NULL, "%s: null output", op);
  DGG_REQUIRE(Sq == 0 || lse2 != nullptr, DGG_ERR_NULL, "%s: null lse pointer", op);
  if (Sq > 0)
    if (int rc = validate_exp_rand(op, exp_rand, er_strides, Sq, tau)) return rc;
  // The row lse of the perturbed scores is base 2 (as dgg_attn_kf_rowlse writes it).
  AttnParams p = make_params(q, k, nullptr, nullptr, B, Sq, Sk, Hq, Hkv, D, scale, 0.f, window,
                             flags | DGG_ATTN_LSE_BASE2);
  p.lse = const_cast<float*>(lse2);
  p.colsum = kf_score;
  p.q_sb = strides[0]; p.q_ss = strides[1]; p.q_sh = strides[2];
  p.k_sb = strides[3]; p.k_ss = strides[4]; p.k_sh = strides[5];
  if (Sq > 0) set_exp_rand(p, exp_rand, er_strides, tau);
  const int64_t bk = D == 128 ? kC128BK : kCBK;
  p.n_tiles = (int)((Sk + bk - 1) / bk);
  const bool ref = (flags & DGG_ATTN_REF_ROUNDING) != 0;
  hipStream_t st = dgg::as_stream(stream);
  if (dtype == DGG_BF16) {
    if (D == 64) pick_col<BF16, 64>(p, ref, kColKF, st);
    else if (D == 128) pick_col<BF16, 128>(p, ref, kColKF, st);
    else pick_col<BF16, 256>(p, ref, kColKF, st);
  } else {
    if (D == 64) pick_col<F16, 64>(p, ref, kColKF, st);
    else if (D == 128) pick_col<F16, 128>(p, ref, kColKF, st);
    else pick_col<F16, 256>(p, ref, kColKF, st);
  }
  return dgg::check_launch(op);
}

extern "C" int dgg_attn_colsum(const void* q, const void* k, const float* lse, float* colsum, int64_t B, int64_t Sq,
                               int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides, float scale,
                               float softcap, int64_t window, uint32_t flags, int dtype, void* stream) {
  return colscore("attn_colsum", q, k, lse, kColSum, colsum, nullptr, nullptr, nullptr, 0, B, Sq, Sk, Hq, Hkv, D, strides,
                  scale, softcap, window, flags, dtype, stream);
}

extern "C" int dgg_attn_colscore(const void* q, const void* k, const float* lse, int epilogue, float* out0, float* out1,
                                 uint8_t* out_any, const float* thr, int64_t thr_row_stride, int64_t B, int64_t Sq,
                                 int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D, const int64_t* strides, float scale,
                                 float softcap, int64_t window, uint32_t flags, int dtype, void* stream) {
  return colscore("attn_colscore", q, k, lse, epilogue, out0, out1, out_any, thr, thr_row_stride, B, Sq, Sk, Hq, Hkv,
                  D, strides, scale, softcap, window, flags, dtype, stream);
}
