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
  const float* er;       // KeyFormer exp_rand [B, Hq, Sq, Sk], element strides er_sb, er_sh, er_ss (unit key stride)
  int64_t er_sb, er_sh, er_ss;
  float kf_inv_tau;      // 1 / tau of the perturbed softmax
  int er_lane32;         // (132 * er_ss + Sk) * 4 < 2^31: the exp_rand byte offsets within a tile fit 32 bits
  int thr_lane32;        // (132 * thr_rs + Sk) * 4 < 2^31: the threshold byte offsets within a tile fit 32 bits
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
  float ref_div;  // the divisor of the reference's scores, fp32: sqrt(D) for the default scale, else 1 / scale
  float ref_rcp;  // RN32(1 / ref_div): torch on the GPU divides a tensor by a Python scalar as x * this
  float c_fast;  // scale * log2(e): converts raw scores to the exp2 domain
  float inv_softcap;
  float softcap;
  float sc_a;    // 2 * scale / softcap * log2(e)
  float sc_b;    // softcap * log2(e)
  const float* rope_cs;  // fused rotary of the query rows: [B * Sq, D] (cos | sin) per row, or nullptr
};

// Probability of the perturbed score for KeyFormer: x2 = the score in the exp2 domain, e = exp_rand, l2 = the
// perturbed row lse in base 2: exp2((x2 - log2 e) / tau - l2) (kf.py:37-39: gumbels = -log(e),
// softmax((scores + gumbels) / tau)).
__device__ __forceinline__ float kf_prob(float x2, float e, float l2, const AttnParams& p) {
  return __builtin_amdgcn_exp2f(fmaf(x2 - __builtin_amdgcn_logf(e), p.kf_inv_tau, -l2));
}

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

// Score transform shared by the forward and column-sum kernels. Returns the value whose exp2 (after the
// row maximum / lse is subtracted and `c` applied) is the unnormalised probability:
//   fast path (no soft-cap, no reference rounding): the raw fp32 score; the caller multiplies by c_fast.
//   otherwise: the score already in the exp2 domain (c = 1).
// REFROUND: the scores are rounded to the input dtype where the reference rounds them (attn.py:29,
// gemma2.py:29-33). Each division by a Python float there (`/ math.sqrt(D)`, `/= softcap`) is what torch executes
// on the GPU for a tensor divided by a CPU scalar: one fp32 multiply by the fp32 reciprocal of the divisor, then
// the rounding to the tensor dtype.
template <typename T, bool SOFTCAP, int REFROUND>
__device__ __forceinline__ float score_value(float s, const AttnParams& p) {
  if constexpr (REFROUND) {
    s = round_t<T>(s);
    s = round_t<T>(s * p.ref_rcp);
    if constexpr (SOFTCAP) {
      s = round_t<T>(s * p.inv_softcap);
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

template <bool SOFTCAP, int REFROUND>
__device__ __forceinline__ float score_coeff(const AttnParams& p) {
  return (SOFTCAP || REFROUND) ? 1.0f : p.c_fast;
}

// Column epilogues of the column-sum kernels: H2O / SnapKV sum p (h2o.py:35-36, snapkv.py:36-37), RoCo also sums
// p^2 (roco.py:43-47), Corm ORs p >= threshold[i][j] over the queries (corm.py:35-37).
// KeyFormer (kf.py:36-40) sums the probabilities of the Gumbel-perturbed scores (s - ln e) / tau instead
// (kColKF: the column kernels then read the perturbed row lse and the exp_rand input e).
enum ColEpi { kColSum = 0, kColSumSq = 1, kColAnyGe = 2, kColKF = 3 };
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
  // Ties the sums so far to this point of the program (a fixed-order schedule would otherwise see its additions
  // sunk past later code that does not use them).
  __device__ __forceinline__ void pin() {
    if constexpr (EPI != kColAnyGe) asm volatile("" : "+v"(s));
    if constexpr (EPI == kColSumSq) asm volatile("" : "+v"(s2));
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
// output rounded to fp16, multiplied by the fp32 reciprocal of the divisor, rounded again (attn.py:29 /
// h2o.py:29 as torch runs them on the GPU). The conversions are v_cvt_pk_f16_f32 and the fp16 operands feed
// v_fma_mix_f32 directly: four instructions per pair.
__device__ __forceinline__ f16x2 ref_scores_f16(float a, float b, const AttnParams& p) {
  const f16x2 h = __builtin_convertvector(f32x2{a, b}, f16x2);
  const float q0 = fmaf((float)h[0], p.ref_rcp, 0.0f);  // +0 addend keeps v_fma_mix (exact: RN32(x * y))
  const float q1 = fmaf((float)h[1], p.ref_rcp, 0.0f);
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

// Forward kernels with grouped query heads (Hq = G * Hkv, G > 1) and B * Hkv divisible by 8: each XCD takes whole
// KV heads, one after the other, and within a KV head the query tiles longest first with the G query heads of a
// tile next to each other. The workgroups resident on an XCD at a time are then adjacent query tiles of the query
// heads of one KV head, whose K/V windows overlap: fewer K/V bytes pass through that XCD's L2 per generation of
// workgroups than with the heads of two KV heads side by side (map_block). Otherwise map_block's order.
__device__ __forceinline__ void map_block_kv(int n_tiles, int B, int Hq, int Hkv, bool reverse, int& tile, int& bh) {
  const int G = Hq / Hkv, nkv = B * Hkv;
  if (G == 1 || (nkv & 7) != 0) return map_block(n_tiles, B * Hq, reverse, tile, bh);
  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  const int per_kv = n_tiles * G;
  const int kv_local = local / per_kv, rem = local - kv_local * per_kv;
  const int t_major = rem / G, qh = rem - t_major * G;
  const int kvi = xcd * (nkv >> 3) + kv_local;  // b * Hkv + hk
  const int b = kvi / Hkv, hk = kvi - b * Hkv;
  bh = b * Hq + hk * G + qh;
  tile = reverse ? n_tiles - 1 - t_major : t_major;
}

// map_block_kv's grouping with a causal sliding window. The first KV head an XCD takes runs its query tiles in
// ascending order: its shorter tiles below the window first (all starting at key 0), then the whole-window tiles,
// each generation of workgroups starting on keys the previous one touched last, which the XCD's L2 still holds.
// A second KV head runs its whole-window tiles (full0 ..) in ascending order and then its shorter tiles longest
// first, so that the XCD's last workgroups are short and the launch ends evenly.
__device__ __forceinline__ void map_block_kv_window(int n_tiles, int B, int Hq, int Hkv, int full0, int& tile,
                                                    int& bh) {
  const int G = Hq / Hkv, nkv = B * Hkv;
  if (G == 1 || (nkv & 7) != 0) return map_block(n_tiles, B * Hq, true, tile, bh);
  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  const int per_kv = n_tiles * G;
  const int kv_local = local / per_kv, rem = local - kv_local * per_kv;
  const int t_major = rem / G, qh = rem - t_major * G;
  const int kvi = xcd * (nkv >> 3) + kv_local;  // b * Hkv + hk
  const int b = kvi / Hkv, hk = kvi - b * Hkv;
  bh = b * Hq + hk * G + qh;
  const int nfull = n_tiles - full0;
  if ((kv_local & 1) == 0) tile = t_major;
  else tile = t_major < nfull ? full0 + t_major : full0 - 1 - (t_major - nfull);
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
// l + the two packed values (one dot-product instruction).
__device__ __forceinline__ float dot2_ones(bf16x2 v, float l) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(v, one, l, false);
}
__device__ __forceinline__ float dot2_ones(f16x2 v, float l) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(v, one, l, false);
}
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


// Host-side validation of the attention arguments shared by the prefill, column and split-KV entry points
// (nstrides strides, every third one a sequence stride), and the launch parameters they derive.
int validate_attn(const char* op, const void* q, const void* k, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq,
                  int64_t Hkv, int64_t D, const int64_t* strides, int nstrides, float scale, float softcap,
                  int64_t window, int dtype);
AttnParams make_params(const void* q, const void* k, const void* v, void* o, int64_t B, int64_t Sq, int64_t Sk,
                       int64_t Hq, int64_t Hkv, int64_t D, float scale, float softcap, int64_t window, uint32_t flags);

// Software-pipelined head_dim-256 forward (attention_d256.hip) for 16-bit inputs without reference rounding:
// 4 waves x 32 rows per workgroup (p.n_tiles counts 128-row query tiles).
void launch_attn_d256_pipe(const AttnParams& p, bool bf16, hipStream_t st);

// fp32 inputs (attention_f32.hip): the forward and the column-score pass, rows per workgroup tile of both.
int f32_rows_per_tile();
void launch_attn_f32_fwd(const AttnParams& p, int D, hipStream_t st);
void launch_attn_f32_col(const AttnParams& p, int D, int epi, hipStream_t st);

}  // namespace dgg_attn
