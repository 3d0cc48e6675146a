// Software-pipelined prefill forward for head_dim 256 on gfx950 (the Gemma-2 case, gemma2.py:19-38: soft-cap,
// sliding window, GQA).
//
// At head_dim 256 a wave's Q fragments (64 registers) and O accumulators (128) leave room for one wave per SIMD,
// so no second wave fills the matrix pipe while a wave runs its soft-cap and softmax. This kernel overlaps the two
// inside the wave instead: iteration t computes the scores of key tile t+1 (S(t+1) = K(t+1) . Q^T, 32 MFMAs)
// while the vector ALU runs the soft-cap and row maximum of tile t, then the P.V product of tile t (32 MFMAs)
// while it runs the exponentials. K and V sit in separate two-slot LDS rings, K one tile ahead of V:
//   iteration t needs K(t+1) (slot (t+1)%2) and V(t) (slot t%2); after its barrier it requests K(t+2) into the
//   K slot that held K(t) and V(t+1) into the V slot that held V(t-1), both finished by every wave.
// One barrier per tile, 4 x 33 KiB of LDS. Tile layout, direct loads and fragment reads are those of the other
// direct-load kernels (attention_common.h, DmaLayout).
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.h"

#include "attention_common.h"
// DGG_D256_WINDOW_ASC (default 1): with a causal sliding window, the query-tile order of map_block_kv_window
// (measured on config 3: 501 MB of L2 misses per launch instead of 571 MB, 0.823-0.827 vs 0.834-0.836 ms); 0 keeps
// the longest-first order for every launch.
#ifndef DGG_D256_WINDOW_ASC
#define DGG_D256_WINDOW_ASC 1
#endif

// DGG_D256_MANUAL (default 1): the fast iterations run the hand-ordered schedule (fast_iter); 0 leaves their order
// to the compiler's scheduler (for A/B measurements).
#ifndef DGG_D256_MANUAL
#define DGG_D256_MANUAL 1
#endif

namespace dgg_attn {
namespace {

template <typename T, bool MASK, bool SOFTCAP, bool FASTSUM>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
attn_fwd_d256_pipe_kernel(AttnParams p) {
  constexpr int D = 256, NW = 4, BN = 64;
  typedef DmaLayout<D> L;
  constexpr int ROW_B = L::ROW_B, GROUP_B = L::GROUP_B, LPR = L::LPR, RPI = L::RPI, IPG = L::IPG;
  typedef typename T::scalar S;
  typedef typename T::vec8 V8;
  typedef typename T::vec4 V4;
  constexpr int TILE_B = (BN / 4) * GROUP_B;  // one K or V tile
  constexpr int GPW = (BN / 4) / NW;          // 4-row groups of a tile copied by each wave
  constexpr int DMA_PER_TILE = GPW * IPG;     // direct loads per wave per K (or V) tile
  constexpr int NMB = BN / 32;                // 32-key blocks per tile
  static_assert(GPW * NW == BN / 4, "tile groups must split over the waves");
  __shared__ __attribute__((aligned(1024))) char smem[4 * TILE_B];  // K slot 0, K slot 1, V slot 0, V slot 1

  constexpr int BM = 32 * NW;  // query rows per workgroup
  int qt, bh;
  if (DGG_D256_WINDOW_ASC && p.causal && p.window > 0) {
    // first query tile whose rows all see a whole window (key of the first row: q0 + offset - window + 1 >= 0)
    const int full0 = min(p.n_tiles, max(0, (p.window - 1 - p.offset + BM - 1) / BM));
    map_block_kv_window(p.n_tiles, p.B, p.Hq, p.Hkv, full0, qt, bh);
  } else {
    map_block_kv(p.n_tiles, p.B, p.Hq, p.Hkv, true, qt, bh);
  }
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / p.group;
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 31, g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qt * BM;
  const int qw0 = q0 + 32 * w;  // first query row of this wave; lane row qw0 + r
  const int qi = qw0 + r;

  const S* qp = static_cast<const S*>(p.q) + b * p.q_sb + h * p.q_sh;
  const char* kp = reinterpret_cast<const char*>(static_cast<const S*>(p.k) + b * p.k_sb + hk * p.k_sh);
  const char* vp = reinterpret_cast<const char*>(static_cast<const S*>(p.v) + b * p.v_sb + hk * p.v_sh);
  const int64_t k_ss_b = p.k_ss * (int64_t)sizeof(S), v_ss_b = p.v_ss * (int64_t)sizeof(S);

  // Q fragments, all loads back to back (a row past the end reads the last row and is zeroed below).
  V8 qf[D / 16];
  {
    const int qr = min(qi, p.Sq - 1);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) qf[kk] = ld16<V8>(qp + (int64_t)qr * p.q_ss + 16 * kk + 8 * g);
  }

  // Key tiles of the workgroup and of this wave.
  const int q_last = min(q0 + BM, p.Sq) - 1;
  int k_begin = 0, k_end = p.Sk;
  if (p.causal) k_end = min(p.Sk, q_last + p.offset + 1);
  if (p.window > 0) k_begin = max(0, q0 + p.offset - p.window + 1);
  const int t_begin = k_begin / BN;
  const int t_end = k_end > k_begin ? (k_end + BN - 1) / BN : t_begin;
  const int wq_last = min(qw0 + 32, p.Sq) - 1;
  int wk_begin = 0, wk_end = p.Sk;
  if (p.causal) wk_end = min(p.Sk, wq_last + p.offset + 1);
  if (p.window > 0) wk_begin = max(0, qw0 + p.offset - p.window + 1);
  // A wave whose rows all lie past the end computes no tile (it still copies its share and meets the barriers).
  const int wt_begin = wk_begin / BN;
  const int wt_end = qw0 < p.Sq && wk_end > wk_begin ? (wk_end + BN - 1) / BN : wt_begin;
  // [t_full0, t_full1): tiles every row of this wave sees whole (no per-element mask).
  int t_full0 = wt_begin, t_full1 = wt_end;
  if constexpr (MASK) {
    if (p.window > 0) {
      const int lo_last = wq_last + p.offset - p.window + 1;
      t_full0 = lo_last <= 0 ? wt_begin : min(wt_end, max(wt_begin, (lo_last + BN - 1) / BN));
    }
    if (p.causal) {
      const int hi_first = qw0 + p.offset;
      t_full1 = max(t_full0, min(wt_end, hi_first < 0 ? wt_begin : (hi_first + 1) / BN));
    }
  }
  if (t_full1 > t_full0 && t_full1 * BN > p.Sk) t_full1 = max(t_full0, p.Sk / BN);
  if (t_full1 < t_full0) t_full1 = t_full0;

  // Visible keys of this lane's row: k_lo <= key <= k_hi.
  int k_hi = p.Sk - 1, k_lo = 0;
  if (p.causal) k_hi = min(k_hi, qi + p.offset);
  if (p.window > 0) k_lo = max(k_lo, qi + p.offset - p.window + 1);

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
  // Ring slots are numbered from the workgroup's first tile: tile t sits in slot (t - t_begin) % 2 of its ring.
  const uint32_t smem_base = (uint32_t)(size_t)((lds_char*)smem);
  constexpr uint32_t V_RING = 2 * TILE_B;

  // Copies this wave's groups GPW*w .. GPW*w + GPW-1 of K (or V) tile t: DMA_PER_TILE loads.
  auto issue = [&](int t, const char* base, int64_t ss_b, const uint32_t* voff, uint32_t dst_slot) {
    const uint32_t dst = dst_slot + (uint32_t)(GPW * w * GROUP_B);
    const int row0 = t * BN + 4 * GPW * w;
    if ((t + 1) * BN <= p.Sk) {
      const char* rb = base + (int64_t)row0 * ss_b;
#pragma unroll
      for (int j = 0; j < GPW; ++j)
#pragma unroll
        for (int i = 0; i < IPG; ++i) dma16(dst + j * GROUP_B + i * RPI * ROW_B, rb + 4 * j * ss_b, voff[i]);
    } else {  // ragged last tile: rows past the end re-read the last row (always masked, finite)
#pragma unroll
      for (int j = 0; j < GPW; ++j)
#pragma unroll
        for (int i = 0; i < IPG; ++i) {
          const int64_t row = min(row0 + 4 * j + i * RPI + lane / LPR, p.Sk - 1);
          dma16(dst + j * GROUP_B + i * RPI * ROW_B, base + row * ss_b + src_chunk[i] * 16);
        }
    }
  };
  auto issue_k = [&](int t, int slot) { issue(t, kp, k_ss_b, k_voff, smem_base + slot * TILE_B); };
  auto issue_v = [&](int t, int slot) { issue(t, vp, v_ss_b, v_voff, smem_base + V_RING + slot * TILE_B); };

  // LDS read addressing, as the other direct-load kernels: K fragment (row mb*32 + r, chunk 2kk + g) at
  // lane part + 64*((kk/2) ^ (r%4)) + constant; V transposing read (rows 16kk + 4g + (lane%16)/4 (+8), head-dim
  // column db*32 + 16*((lane/16)%2) + 4*(lane%4)) at lane part + 64*(db ^ (lane%16)/4) + constant. The swizzle
  // flips the low two bits of the 64-byte column index only, so i ^ s = 4*(i/4) + ((i%4) ^ s): four base
  // registers per ring plus the slot offset, and the rest of each address (4*(i/4), block, step) is an immediate.
  const int s4 = r & 3;
  const uint32_t k_lane = (uint32_t)((r >> 2) * GROUP_B + s4 * ROW_B + 16 * g);
  const int m4 = (lane & 15) >> 2, m3 = lane & 3;
  const uint32_t v_lane = (uint32_t)(g * GROUP_B + m4 * ROW_B + 32 * ((lane >> 4) & 1) + 16 * (m3 >> 1) + 8 * (m3 & 1));
  uint32_t kb[4], vb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kb[i] = smem_base + k_lane + 64u * (uint32_t)(i ^ s4);
    vb[i] = smem_base + V_RING + v_lane + 64u * (uint32_t)(i ^ m4);
    asm volatile("" : "+v"(kb[i]), "+v"(vb[i]));
  }

  f32x16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) oacc[i] = f32x16{};
  float m_run = -INFINITY, l_part[2] = {0.f, 0.f};
  const float c = score_coeff<SOFTCAP, 0>(p);

  // S^T = K . Q^T of the tile in K slot `slot` into s (one query per lane, the keys of 32-key block mb in s[mb]).
  auto qk = [&](const uint32_t slot, f32x16 (&s)[NMB]) __attribute__((always_inline)) {
    uint32_t kbs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kbs[i] = kb[i] + slot * TILE_B;
      asm volatile("" : "+v"(kbs[i]));  // one add per base and tile, not one per read
    }
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) s[mb] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const int i = kk >> 1;
        const V8 a = lds_read<V8>(kbs[i & 3] + 256 * (i >> 2) + mb * 8 * GROUP_B + 32 * (kk & 1));
        s[mb] = mfma32(a, qf[kk], s[mb]);
      }
  };

  // Folds a tile's row maximum (this lane's part) into m_run; rescales O and l when the maximum grows past the
  // lazy threshold (after the P.V products issued before it, which the rescale waits for).
  auto fold_max = [&](float mloc) __attribute__((always_inline)) {
    mloc = half_swap_max(mloc);
    const float m_new = fmaxf(m_run, mloc);
    const bool need = m_new * c > m_run * c + kRescaleThreshold;
    if (__any(need)) {
      const float alpha = need ? fast_exp2((m_run - m_new) * c) : 1.0f;
      if (need) m_run = m_new;
      l_part[0] *= alpha;
      l_part[1] *= alpha;
#pragma unroll
      for (int i = 0; i < D / 32; ++i) oacc[i] *= alpha;
    }
  };

  // Prepared form of a score. Without a soft-cap: the raw score x (its exp2-domain value is x * c). With one: the
  // soft-cap's reciprocal r = 1 / (exp2(s * sc_a) + 1), of which the exp2-domain value x = sc_b - 2 sc_b r
  // (softcap * tanh(s * scale / softcap) * log2(e)) is a decreasing function. The row maximum is then tracked as the
  // minimum r, and the exponent x - m is one fma of r, so x itself is never formed. Masked scores: -inf / +inf.
  const float sc_m2 = -2.0f * p.sc_b;
  constexpr float MASKED_VAL = SOFTCAP ? INFINITY : -INFINITY;
  // (With a soft-cap Q is pre-scaled by sc_a when it is loaded, so the MFMA yields s * sc_a directly; the scaled Q
  // is rounded to the input dtype, a relative 2^-9 (bf16) of each score, as the reference's own rounding of the
  // scores to the input dtype.)
  auto prep_val = [&](float sraw) __attribute__((always_inline)) {
    if constexpr (SOFTCAP) return fast_rcp(fast_exp2(sraw) + 1.0f);
    else return sraw;
  };
  auto ext_upd = [&](float acc, float v) __attribute__((always_inline)) {
    if constexpr (SOFTCAP) return fminf(acc, v);
    else return fmaxf(acc, v);
  };
  auto ext_to_max = [&](float acc) __attribute__((always_inline)) {  // the row maximum (exp2 domain / c)
    if constexpr (SOFTCAP) return fmaf(acc, sc_m2, p.sc_b);
    else return acc;
  };

  // Soft-cap, mask and row maximum of tile t in s, folded into m_run.
  auto prep = [&](const int t, f32x16 (&s)[NMB], auto masked) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked)::value;
    const int kb4 = t * BN + 4 * g;
    const int rel_hi = k_hi - kb4, rel_lo = k_lo - kb4;
    float ext = MASKED_VAL;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float x = prep_val(s[mb][j]);
        if constexpr (MASKED) {
          const int o = mb * 32 + 8 * (j >> 2) + (j & 3);
          x = (o <= rel_hi && o >= rel_lo) ? x : MASKED_VAL;
        }
        s[mb][j] = x;
        ext = ext_upd(ext, x);
      }
    fold_max(ext_to_max(ext));
  };
  // exp2-domain exponent of a prepared score relative to the row's reference maximum: x * c - m * c; mcb is
  // m * c (soft-cap: sc_b - m, c = 1).
  auto rel_exp = [&](float v, float mcb) __attribute__((always_inline)) {
    if constexpr (SOFTCAP) return fmaf(v, sc_m2, mcb);
    else return fmaf(v, c, -mcb);
  };
  auto row_mcb = [&]() __attribute__((always_inline)) {
    const float mc = m_run == -INFINITY ? 0.f : m_run * c;
    return SOFTCAP ? p.sc_b - mc : mc;
  };

  // P = exp2(x*c - m*c) of a prepared tile, rounded to the storage type (pb[kk]: keys 16kk .. 16kk+15), and the
  // row sums.
  auto expo = [&](const f32x16 (&s)[NMB], V8 (&pb)[BN / 16]) __attribute__((always_inline)) {
    const float mcb = row_mcb();
#pragma unroll
    for (int kk = 0; kk < BN / 16; ++kk) {
      f32x8 pv8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = fast_exp2(rel_exp(s[kk >> 1][8 * (kk & 1) + e], mcb));
        if constexpr (!FASTSUM) l_part[e & 1] += pe;
        pv8[e] = pe;
      }
      pb[kk] = from_f32x8<V8>(pv8);
      if constexpr (FASTSUM) l_part[kk & 1] = rowsum8(pb[kk], l_part[kk & 1]);
    }
  };

  // O^T += V^T . P^T with V in V slot `slot`.
  auto pvmm = [&](const uint32_t slot, const V8 (&pb)[BN / 16]) __attribute__((always_inline)) {
    uint32_t vbs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vbs[i] = vb[i] + slot * TILE_B;
      asm volatile("" : "+v"(vbs[i]));
    }
#pragma unroll
    for (int kk = 0; kk < BN / 16; ++kk)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const uint32_t va = vbs[db & 3] + 256 * (db >> 2) + kk * 4 * GROUP_B;
        const V4 lo = tr_read_at(va, S{});
        const V4 hi = tr_read_at(va + 2 * GROUP_B, S{});
        const V8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[db] = mfma32(a, pb[kk], oacc[db]);
      }
  };

  // The fast iteration in a fixed order, one step per MFMA, each step fenced (sched_barrier) so that the compiler
  // keeps it. Steps 0-31: K fragment read two steps ahead, one QK^T MFMA of tile t+1, the exponential of one
  // element of tile t (fma + exp; every second step the pair's conversion and row-sum dot2). Steps 32-63: V^T
  // fragment reads two steps ahead, one P.V MFMA of tile t, the soft-cap and maximum of one element of tile t+1.
  // cur: the ring slot of tile t (K of t+1 in the other K slot).
  typedef typename std::conditional<std::is_same<T, BF16>::value, bf16x2, f16x2>::type H2;
  // The copies of K(t+2) and V(t+1) (whole tiles in every fast iteration) are issued one per step over steps 0-15,
  // so that their issue overlaps the MFMAs.
  auto fast_iter = [&](const uint32_t cur, const int t, f32x16 (&sc)[NMB], f32x16 (&sn)[NMB])
      __attribute__((always_inline)) {
    constexpr int PF = 2;  // fragment prefetch distance, in steps
    const char* krow = kp + (int64_t)((t + 2) * BN + 4 * GPW * w) * k_ss_b;
    const char* vrow = vp + (int64_t)((t + 1) * BN + 4 * GPW * w) * v_ss_b;
    const uint32_t kdst = smem_base + cur * TILE_B + (uint32_t)(GPW * w * GROUP_B);
    const uint32_t vdst = smem_base + V_RING + (cur ^ 1u) * TILE_B + (uint32_t)(GPW * w * GROUP_B);
    uint32_t kbs[4], vbs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kbs[i] = kb[i] + (cur ^ 1u) * TILE_B;
      vbs[i] = vb[i] + cur * TILE_B;
      asm volatile("" : "+v"(kbs[i]), "+v"(vbs[i]));
    }
    auto kaddr = [&](int i) {
      const int kk = i >> 1, mb = i & 1, ii = kk >> 1;
      return kbs[ii & 3] + 256 * (ii >> 2) + mb * 8 * GROUP_B + 32 * (kk & 1);
    };
    auto vaddr = [&](int i) {
      const int kk = i >> 3, db = i & 7;
      return vbs[db & 3] + 256 * (db >> 2) + kk * 4 * GROUP_B;
    };
    const float mcb = row_mcb();
    V8 ka[PF + 1];
#pragma unroll
    for (int i = 0; i < PF; ++i) ka[i] = lds_read<V8>(kaddr(i));
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) sn[mb] = f32x16{};
    H2 pw[BN / 16][4];  // P of tile t as packed pairs: pw[kk][q] = keys 16kk + {2q, 2q+1} of the B operand order
    float pe_even = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (i < DMA_PER_TILE) {
        const int j = i / IPG, ii = i % IPG;
        dma16(kdst + j * GROUP_B + ii * RPI * ROW_B, krow + 4 * j * k_ss_b, k_voff[ii]);
      } else if (i < 2 * DMA_PER_TILE) {
        const int j = (i - DMA_PER_TILE) / IPG, ii = (i - DMA_PER_TILE) % IPG;
        dma16(vdst + j * GROUP_B + ii * RPI * ROW_B, vrow + 4 * j * v_ss_b, v_voff[ii]);
      }
      if (i + PF < 32) ka[(i + PF) % (PF + 1)] = lds_read<V8>(kaddr(i + PF));
      sn[i & 1] = mfma32(ka[i % (PF + 1)], qf[i >> 1], sn[i & 1]);
      const int kk = i >> 3, e = i & 7;
      const float pe = fast_exp2(rel_exp(sc[kk >> 1][8 * (kk & 1) + e], mcb));
      if constexpr (!FASTSUM) l_part[e & 1] += pe;
      if (e & 1) {
        pw[kk][e >> 1] = __builtin_convertvector(f32x2{pe_even, pe}, H2);
        if constexpr (FASTSUM) l_part[kk & 1] = dot2_ones(pw[kk][e >> 1], l_part[kk & 1]);
      } else {
        pe_even = pe;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    V8 pb[BN / 16];
#pragma unroll
    for (int kk = 0; kk < BN / 16; ++kk)
      pb[kk] = __builtin_shufflevector(__builtin_shufflevector(pw[kk][0], pw[kk][1], 0, 1, 2, 3),
                                       __builtin_shufflevector(pw[kk][2], pw[kk][3], 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
    V4 va[PF + 1][2];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      va[i][0] = tr_read_at(vaddr(i), S{});
      va[i][1] = tr_read_at(vaddr(i) + 2 * GROUP_B, S{});
    }
    float ext = MASKED_VAL;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (i + PF < 32) {
        va[(i + PF) % (PF + 1)][0] = tr_read_at(vaddr(i + PF), S{});
        va[(i + PF) % (PF + 1)][1] = tr_read_at(vaddr(i + PF) + 2 * GROUP_B, S{});
      }
      const V8 a = __builtin_shufflevector(va[i % (PF + 1)][0], va[i % (PF + 1)][1], 0, 1, 2, 3, 4, 5, 6, 7);
      oacc[i & 7] = mfma32(a, pb[i >> 3], oacc[i & 7]);
      const float x = prep_val(sn[i >> 4][i & 15]);
      sn[i >> 4][i & 15] = x;
      ext = ext_upd(ext, x);
      __builtin_amdgcn_sched_barrier(0);
    }
    fold_max(ext_to_max(ext));
  };

  // Pipeline iteration t (on entry tile t is prepared in scur: soft-capped, masked, its maximum folded into m_run):
  // the barrier, the copies of K(t+2) and V(t+1); then the scores of tile t+1 under the exponentials of tile t, and
  // the P.V product of tile t under the soft-cap and row maximum of tile t+1. FAST: this wave sees tile t and sees
  // tile t+1 whole, so each pair runs in one block and the scheduler interleaves the MFMAs with the vector work.
  auto iter = [&](const int t, auto fast, f32x16 (&sc)[NMB], f32x16 (&sn)[NMB]) __attribute__((always_inline)) {
    const uint32_t cur = (uint32_t)(t - t_begin) & 1u;
    wait_vmem<0>();
    __syncthreads();
    constexpr bool FAST = decltype(fast)::value;
    // the fast schedule issues its own copies (whole tiles K(t+2) and V(t+1), see fb below)
    if (!(FAST && DGG_D256_MANUAL)) {
      if (t + 2 < t_end) issue_k(t + 2, cur);
      if (t + 1 < t_end) issue_v(t + 1, cur ^ 1u);
    }
    V8 pb[BN / 16];
    if constexpr (FAST && DGG_D256_MANUAL) {
      fast_iter(cur, t, sc, sn);
    } else if constexpr (FAST) {
      qk(cur ^ 1u, sn);
      expo(sc, pb);
      pvmm(cur, pb);
      prep(t + 1, sn, std::false_type{});
    } else {
      const bool do_qk = t + 1 >= wt_begin && t + 1 < wt_end;
      if (do_qk) qk(cur ^ 1u, sn);
      if (t >= wt_begin && t < wt_end) {
        expo(sc, pb);
        pvmm(cur, pb);
      }
      if (do_qk) {
        if (t + 1 >= t_full0 && t + 1 < t_full1) prep(t + 1, sn, std::false_type{});
        else prep(t + 1, sn, std::true_type{});
      }
    }
  };

  f32x16 scur[NMB], snext[NMB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) scur[mb] = snext[mb] = f32x16{};
  if (t_begin < t_end) {
    issue_k(t_begin, 0);
    if (t_begin + 1 < t_end) issue_k(t_begin + 1, 1);
    issue_v(t_begin, 0);
    // Q: zero the rows past the end, pin the fragments in AGPRs (MFMA reads its B operand from there; the VGPRs
    // stay free for O, the two score tiles and the fragments read ahead).
    const bool live = qi < p.Sq;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      asm volatile("" : "+v"(qf[kk]));
      if (!live) qf[kk] = V8{};
      if constexpr (SOFTCAP) qf[kk] = from_f32x8<V8>(to_f32x8(qf[kk]) * p.sc_a);
      asm volatile("" : "+a"(qf[kk]));
    }
    if (t_begin + 1 < t_end) wait_vmem<2 * DMA_PER_TILE>();  // K(t_begin) has landed
    else wait_vmem<DMA_PER_TILE>();
    __syncthreads();
    if (t_begin >= wt_begin && t_begin < wt_end) {
      qk(0u, scur);
      if (t_begin >= t_full0 && t_begin < t_full1) prep(t_begin, scur, std::false_type{});
      else prep(t_begin, scur, std::true_type{});
    }
    // [t_begin, fa) and [fb, t_end) one tile at a time; [fa, fb) the fast iterations (every wave runs every t, one
    // barrier each, so the barrier counts agree).
    const int fa = min(max(max(t_full0 - 1, wt_begin), t_begin), t_end);
    // (fast iterations also copy K(t+2) and V(t+1) as whole tiles: t + 2 < t_end and (t + 3) * BN <= Sk)
    const int fb = max(fa, min(min(t_full1 - 1, wt_end - 1), min(t_end - 2, p.Sk / BN - 2)));
    // After each iteration the next tile's scores move into scur (a swap of the two buffers in an unrolled loop
    // measured no faster and pushed the register allocation into spills).
    auto copy_next = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) scur[mb] = snext[mb];
    };
    int t = t_begin;
    for (; t < fa; ++t) {
      iter(t, std::false_type{}, scur, snext);
      copy_next();
    }
    for (; t < fb; ++t) {
      iter(t, std::true_type{}, scur, snext);
      copy_next();
    }
    for (; t < t_end; ++t) {
      iter(t, std::false_type{}, scur, snext);
      copy_next();
    }
  }

  const float l_tot = half_swap_sum(l_part[0] + l_part[1]);
  const float inv = p.Sk == 0 ? 0.f : 1.0f / l_tot;  // no keys at all: o = 0 (an empty P.V), lse = -inf
  if (qi < p.Sq) {
    S* op = static_cast<S*>(p.o) + b * p.o_sb + (int64_t)qi * p.o_ss + h * p.o_sh;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
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

template <typename T, bool MASK, bool SOFTCAP>
void launch(const AttnParams& p, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  if (p.lse == nullptr)
    hipLaunchKernelGGL((attn_fwd_d256_pipe_kernel<T, MASK, SOFTCAP, true>), dim3(grid), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((attn_fwd_d256_pipe_kernel<T, MASK, SOFTCAP, false>), dim3(grid), dim3(256), 0, st, p);
}

}  // namespace

void launch_attn_d256_pipe(const AttnParams& p, bool bf16, hipStream_t st) {
  const bool mask = p.causal || p.window > 0;
  const bool sc = p.softcap > 0.f;
  if (bf16) {
    if (mask) sc ? launch<BF16, true, true>(p, st) : launch<BF16, true, false>(p, st);
    else sc ? launch<BF16, false, true>(p, st) : launch<BF16, false, false>(p, st);
  } else {
    if (mask) sc ? launch<F16, true, true>(p, st) : launch<F16, true, false>(p, st);
    else sc ? launch<F16, false, true>(p, st) : launch<F16, false, false>(p, st);
  }
}

}  // namespace dgg_attn
