// Device-side building blocks of the attention kernels (attention.hip): the launch parameters, MFMA / LDS helpers,
// the score transforms of the reference's rounding and soft-cap modes, the workgroup-to-tile mapping, the
// direct-to-LDS copy helpers and the cross-half / packed row reductions.
#pragma once

#include <algorithm>
#include <type_traits>

#include "common.h"

namespace dgg_attn {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 32 * kWaves;  // query rows per forward workgroup
constexpr float kRescaleThreshold = 8.0f;  // log2 units


struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  float* colsum;
  float* colsum2;        // column sums of p^2 (kColSumSq)
  const float* thr;      // [Sq, Sk] thresholds, row stride thr_rs (kColAnyGe)
  int64_t thr_rs;
  uint8_t* any_out;      // [B, Hq, Sk] (kColAnyGe)
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int B, Sq, Sk, Hq, Hkv, group;
  int n_tiles;   // forward: query tiles; colsum: key tiles
  int causal;
  int window;    // 0 = none
  int offset;    // Sk - Sq (bottom-right aligned causal mask)
  int lse_base2;  // lse written / read in base 2 (DGG_ATTN_LSE_BASE2)
  float scale;
  float ref_div;  // 1 / scale rounded to fp32 (== fp32 sqrt(D) for the usual scale): the reference divides
                  // the rounded scores by it
  float ref_rcp;  // 1 / ref_div rounded to fp32
  float c_fast;  // scale * log2(e): converts raw scores to the exp2 domain
  float inv_softcap;
  float softcap;
  float sc_a;    // 2 * scale / softcap * log2(e)
  float sc_b;    // softcap * log2(e)
};

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16). Within each group of 16 lanes, lane m supplies the address
// of 4 consecutive 16-bit elements M[m][0..3]; lane j receives M[4e + j/4][j%4] for e = 0..3.
__device__ __forceinline__ bf16x4 tr_read(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((bf16x4 __attribute__((address_space(3)))*)(p));
}
typedef __fp16 fp16x4_builtin __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f16x4 tr_read(const _Float16* p) {
  return __builtin_bit_cast(
      f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4_builtin __attribute__((address_space(3)))*)(p)));
}

template <typename T>
__device__ __forceinline__ float round_t(float x) {
  return to_f<typename T::scalar>(to_s<typename T::scalar>(x));
}

// x / d for the reference-rounding mode, from y = RN(1/d): q = RN(x*y), r = x - q*d (exact in one fma),
// q' = RN(q + r*y). By Markstein's theorem (y within half an ulp of 1/d, q within one ulp of x/d) q' is the
// correctly rounded quotient RN(x/d) whenever no intermediate underflows or overflows. Every caller rounds
// q' on to fp16 / bf16 at once; checked exhaustively over all 2^16 fp16 and bf16 x for the usual divisors
// and 200 random ones in [0.01, 1000] (tests/test_ref_division.py), the rounded results equal those of the
// true division (up to the sign of a zero quotient, which no later step sees). The clamp keeps x = +-inf (a
// score that overflowed fp16) from turning into inf - inf: it yields +-inf like the division does. Three
// fma-class instructions and a clamp instead of the ~10 of the IEEE division sequence.
__device__ __forceinline__ float ref_quot(float x, float d, float y) {
  float q = fmaf(x, y, 0.0f);  // +0 addend keeps v_fma_mix (a -0 addend folds to a plain multiply)
  q = __builtin_amdgcn_fmed3f(q, -3.402823466e38f, 3.402823466e38f);
  const float r = fmaf(-q, d, x);
  return fmaf(r, y, q);
}

// Score transform shared by the forward and column-sum kernels. Returns the value whose exp2 (after the
// row maximum / lse is subtracted and `c` applied) is the unnormalised probability:
//   fast path (no soft-cap, no reference rounding): the raw fp32 score; the caller multiplies by c_fast.
//   otherwise: the score already in the exp2 domain (c = 1).
template <typename T, bool SOFTCAP, bool REFROUND>
__device__ __forceinline__ float score_value(float s, const AttnParams& p) {
  if constexpr (REFROUND) {
    // deepgengraph_exp/cases/kernels/attn.py:29 / gemma2.py:29-33: each step rounded to the input dtype;
    // `/ math.sqrt(D)` is an fp32 true division before the rounding.
    s = round_t<T>(s);
    s = round_t<T>(ref_quot(s, p.ref_div, p.ref_rcp));
    if constexpr (SOFTCAP) {
      s = round_t<T>(ref_quot(s, p.softcap, p.inv_softcap));
      s = round_t<T>(tanhf(s));
      s = round_t<T>(s * p.softcap);
    }
    return s * kLog2e;
  } else if constexpr (SOFTCAP) {
    // softcap * tanh(s * scale / softcap) in the exp2 domain, tanh(y) = 1 - 2 / (exp(2y) + 1).
    const float e = fast_exp2(s * p.sc_a);
    return fmaf(fast_rcp(e + 1.0f), -2.0f * p.sc_b, p.sc_b);
  } else {
    return s;
  }
}

template <bool SOFTCAP, bool REFROUND>
__device__ __forceinline__ float score_coeff(const AttnParams& p) {
  return (SOFTCAP || REFROUND) ? 1.0f : p.c_fast;
}

// Column epilogues of the column-sum kernels: H2O / SnapKV sum p (h2o.py:35-36, snapkv.py:36-37), RoCo also sums
// p^2 (roco.py:43-47), Corm ORs p >= threshold[i][j] over the queries (corm.py:35-37).
enum ColEpi { kColSum = 0, kColSumSq = 1, kColAnyGe = 2 };
template <int EPI>
struct ColAcc {
  float s = 0.f, s2 = 0.f;
  int any = 0;
  // p of (query row qi, this lane's key kj); valid = qi < Sq (rows past the end take no part)
  __device__ __forceinline__ void add(float pe, bool valid, int qi, int kjc, const AttnParams& p) {
    if constexpr (EPI == kColAnyGe) {
      if (valid) any |= pe >= p.thr[(int64_t)qi * p.thr_rs + kjc];
    } else {
      s += pe;
      if constexpr (EPI == kColSumSq) s2 = fmaf(pe, pe, s2);
    }
  }
  // Combines the two lane halves (rows 4g..) and stores column kj of (batch, head) bh.
  __device__ __forceinline__ void store(const AttnParams& p, int bh, int kj, int g) {
    if constexpr (EPI == kColAnyGe) {
      const int a = any | __shfl_xor(any, 32, 64);
      if (g == 0 && kj < p.Sk) p.any_out[(int64_t)bh * p.Sk + kj] = (uint8_t)(a != 0);
    } else {
      s += __shfl_xor(s, 32, 64);
      if constexpr (EPI == kColSumSq) s2 += __shfl_xor(s2, 32, 64);
      if (g == 0 && kj < p.Sk) {
        p.colsum[(int64_t)bh * p.Sk + kj] = s;
        if constexpr (EPI == kColSumSq) p.colsum2[(int64_t)bh * p.Sk + kj] = s2;
      }
    }
  }
};

// Reference-rounded fp16 scores of two raw fp32 dot products, kept packed (natural-log domain): the matmul
// output rounded to fp16, divided by ref_div, rounded again (attn.py:29 / h2o.py:29). The conversions are
// v_cvt_pk_f16_f32 and the fp16 operands feed v_fma_mix_f32 directly, so the pair costs ten instructions.
__device__ __forceinline__ f16x2 ref_scores_f16(float a, float b, const AttnParams& p) {
  const f16x2 h = __builtin_convertvector(f32x2{a, b}, f16x2);
  const float q0 = ref_quot((float)h[0], p.ref_div, p.ref_rcp);
  const float q1 = ref_quot((float)h[1], p.ref_div, p.ref_rcp);
  return __builtin_convertvector(f32x2{q0, q1}, f16x2);
}

// Maps blockIdx.x to (tile, batch*head). Longest tiles first; when the (batch, head) count divides by 8,
// each XCD gets a contiguous group of heads so their K/V are shared through that XCD's L2.
__device__ __forceinline__ void map_block(int n_tiles, int bh_count, bool reverse, int& tile, int& bh) {
  const int bid = blockIdx.x;
  int t_major, bh_minor;
  if ((bh_count & 7) == 0) {
    const int hpx = bh_count >> 3;
    const int xcd = bid & 7, local = bid >> 3;
    t_major = local / hpx;
    bh_minor = xcd * hpx + (local - t_major * hpx);
  } else {
    t_major = bid / bh_count;
    bh_minor = bid - t_major * bh_count;
  }
  tile = reverse ? n_tiles - 1 - t_major : t_major;
  bh = bh_minor;
}

// ------------------------------------------------------------------------------------------------
// Forward kernel.
// ------------------------------------------------------------------------------------------------
template <typename T, int D, int BN, bool MASK, bool SOFTCAP, bool REFROUND>
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
  auto step = [&](const int t, auto masked) {
    const int buf = (t - t_begin) & 1;
    const int tn = t + 1;
    const bool prefetch = tn < t_end && tile_full(tn);
    if (prefetch) load_full();
    tile(t, buf, masked);
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
  const float inv = 1.0f / l_tot;
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
// Forward kernel for head_dim 128 and 256 ("DMA kernel"). NW waves of 32*NQB query rows each; K/V tiles of BN
// keys are copied global -> LDS by the direct-to-LDS loads of gfx950 (no VGPR staging, no LDS store
// instructions) into an NSTAGE ring, with one barrier per tile. head_dim 128 runs 8 waves at two per SIMD;
// head_dim 256 (Q 64 + O 128 VGPRs per lane) runs 4 waves at one per SIMD. Each 16-byte chunk c of tile row r
// sits at
//     (r/4)*GROUP_B + (r%4)*ROW_B + 16*(c ^ 4*(r%4))        (ROW_B = 2*D bytes, 4-row groups padded by 16 bytes)
// which keeps both the K fragment reads (16 lanes, 16 rows, one chunk) and the V transposing reads (4 rows x
// 4 chunks per 16-lane group) on distinct LDS banks; the direct loads write that layout by fetching, for LDS
// position p of a row, global chunk p ^ 4*(r%4). One direct load covers 1 KiB: 4 rows of 128 or 2 of 256.
// ------------------------------------------------------------------------------------------------
template <int D>
struct DmaLayout {
  static constexpr int ROW_B = D * 2;             // bytes per K/V row
  static constexpr int GROUP_B = 4 * ROW_B + 16;  // 4-row group + pad
  static constexpr int LPR = ROW_B / 16;          // lanes per row in one direct load
  static constexpr int RPI = 64 / LPR;            // rows per direct load
  static constexpr int IPG = 4 / RPI;             // direct loads per 4-row group
};

typedef __attribute__((address_space(3))) char lds_char;

template <typename V>
__device__ __forceinline__ V lds_read(uint32_t addr) {
  return *reinterpret_cast<const V __attribute__((address_space(3)))*>((lds_char*)(size_t)addr);
}
__device__ __forceinline__ bf16x4 tr_read_at(uint32_t addr, __bf16) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((bf16x4 __attribute__((address_space(3)))*)(size_t)addr);
}
__device__ __forceinline__ f16x4 tr_read_at(uint32_t addr, _Float16) {
  return __builtin_bit_cast(
      f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((fp16x4_builtin __attribute__((address_space(3)))*)(size_t)addr));
}

// Direct global -> LDS copy (global_load_lds_dwordx4): lane l's 16 bytes land at LDS byte address lds + 16*l.
// The copy is not tracked by the compiler's wait counting; callers wait with wait_vmem().
__device__ __forceinline__ void dma16(uint32_t lds, const void* sbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(sbase)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16(uint32_t lds, const void* vaddr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(vaddr)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Cross-half (lanes l and l ^ 32) max / sum of a wave64 value, without an LDS round trip.
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Row-sum accumulation of 8 packed probabilities: l += sum of the rounded values, two per dot-product instruction.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float rowsum8(bf16x8 v, float l) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), one, l, false);
  l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), one, l, false);
  l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), one, l, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), one, l, false);
}
__device__ __forceinline__ float rowsum8(f16x8 v, float l) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  l = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 0, 1), one, l, false);
  l = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 2, 3), one, l, false);
  l = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 4, 5), one, l, false);
  return __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 6, 7), one, l, false);
}


}  // namespace dgg_attn
