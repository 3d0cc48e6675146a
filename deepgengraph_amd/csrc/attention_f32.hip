// fp32 attention: the forward (O and lse) and the column-score pass of the selection cases for fp32 inputs, the
// dtype of config 1 and of any case module the caller runs in fp32 (the reference's modules take any float
// dtype: attn.py:18-34 computes in the input dtype, so fp32 inputs give fp32 scores, an fp32 softmax and an fp32
// P.V with no 16-bit rounding anywhere).
//
// These kernels are the plumbing path, not a tuned one: fp32 has no MFMA at the 16-bit rate, and the fp32
// workloads of the reference are small. Four adjacent lanes share one query row (forward) or one key (column
// pass), each holding a quarter of the head dimension in registers; the dot products are reduced over the four
// lanes with two cross-lane adds. K/V (forward) or Q and its lse (column pass) are staged through LDS in tiles
// of 32 rows. exp / log are the accurate device expf / logf.
#include "attention_common.h"

namespace dgg_attn {
namespace {

constexpr int kRows = 64;      // query rows (forward) / keys (column pass) per workgroup
constexpr int kThr = 4 * kRows;
constexpr int kTile = 32;      // keys (forward) / query rows (column pass) per LDS tile

// Dot product of this lane's quarter with quarter `qd` of an LDS row, summed over the four lanes of the quad.
template <int D>
__device__ __forceinline__ float quad_dot(const float (&a)[D / 4], const float* row) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < D / 4; e += 4) {
    const f32x4 b = *reinterpret_cast<const f32x4*>(row + e);
    s = fmaf(a[e], b[0], s);
    s = fmaf(a[e + 1], b[1], s);
    s = fmaf(a[e + 2], b[2], s);
    s = fmaf(a[e + 3], b[3], s);
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  return s;
}

// The score as the reference computes it in fp32: the matmul result times the fp32 reciprocal of the divisor
// (torch's GPU division by a Python float), then softcap * tanh(s / softcap) (gemma2.py:31-33).
template <bool SOFTCAP>
__device__ __forceinline__ float f32_score(float dot, const AttnParams& p) {
  float s = dot * p.ref_rcp;
  if constexpr (SOFTCAP) s = tanhf(s * p.inv_softcap) * p.softcap;
  return s;
}

// Copies rows r0 .. r0 + kTile - 1 of a [rows, D] fp32 matrix (row stride rs elements) into lds[kTile][D + 4];
// rows at or past n are zero.
template <int D>
__device__ __forceinline__ void stage_rows(float (*lds)[D + 4], const float* src, int64_t rs, int r0, int n) {
  constexpr int C4 = D / 4;  // 16-byte chunks per row
  for (int c = threadIdx.x; c < kTile * C4; c += kThr) {
    const int r = c / C4, col = (c % C4) * 4;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (r0 + r < n) v = *reinterpret_cast<const f32x4*>(src + (int64_t)(r0 + r) * rs + col);
    *reinterpret_cast<f32x4*>(&lds[r][col]) = v;
  }
}

template <int D, bool SOFTCAP>
__global__ void __launch_bounds__(kThr) attn_fwd_f32_kernel(AttnParams p) {
  constexpr int DQ = D / 4;
  __shared__ __attribute__((aligned(16))) float Ks[kTile][D + 4];
  __shared__ __attribute__((aligned(16))) float Vs[kTile][D + 4];
  int qt, bh;
  map_block(p.n_tiles, p.B * p.Hq, true, qt, bh);
  const int b = bh / p.Hq, h = bh - b * p.Hq, hk = h / p.group;
  const int row = threadIdx.x >> 2, qd = threadIdx.x & 3;
  const int q0 = qt * kRows, qi = q0 + row;
  const float* qp = static_cast<const float*>(p.q) + b * p.q_sb + h * p.q_sh;
  const float* kp = static_cast<const float*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const float* vp = static_cast<const float*>(p.v) + b * p.v_sb + hk * p.v_sh;

  float qv[DQ], o[DQ];
  const float* qrow = qp + (int64_t)min(qi, p.Sq - 1) * p.q_ss + qd * DQ;
#pragma unroll
  for (int e = 0; e < DQ; e += 4) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(qrow + e);
    qv[e] = v[0];
    qv[e + 1] = v[1];
    qv[e + 2] = v[2];
    qv[e + 3] = v[3];
  }
#pragma unroll
  for (int e = 0; e < DQ; ++e) o[e] = 0.f;

  // Keys of the workgroup and of this row (bottom-right causal, window).
  const int q_last = min(q0 + kRows, p.Sq) - 1;
  int k_begin = 0, k_end = p.Sk;
  if (p.causal) k_end = min(p.Sk, q_last + p.offset + 1);
  if (p.window > 0) k_begin = max(0, q0 + p.offset - p.window + 1);
  int k_hi = p.Sk - 1, k_lo = 0;
  if (p.causal) k_hi = min(k_hi, qi + p.offset);
  if (p.window > 0) k_lo = max(k_lo, qi + p.offset - p.window + 1);

  float m = -INFINITY, l = 0.f;
  for (int kb = (k_begin / kTile) * kTile; kb < k_end; kb += kTile) {
    __syncthreads();
    stage_rows<D>(Ks, kp, p.k_ss, kb, p.Sk);
    stage_rows<D>(Vs, vp, p.v_ss, kb, p.Sk);
    __syncthreads();
    float s[kTile];
    float mt = -INFINITY;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      const float x = f32_score<SOFTCAP>(quad_dot<D>(qv, &Ks[j][qd * DQ]), p);
      const int key = kb + j;
      s[j] = key >= k_lo && key <= k_hi ? x : -INFINITY;
      mt = fmaxf(mt, s[j]);
    }
    const float m_new = fmaxf(m, mt);
    if (m_new == -INFINITY) continue;  // nothing visible yet
    if (m_new > m) {
      const float alpha = expf(m - m_new);  // 0 while m is -inf
      l *= alpha;
#pragma unroll
      for (int e = 0; e < DQ; ++e) o[e] *= alpha;
      m = m_new;
    }
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      const float pj = expf(s[j] - m);
      l += pj;
      const float* vr = &Vs[j][qd * DQ];
#pragma unroll
      for (int e = 0; e < DQ; ++e) o[e] = fmaf(pj, vr[e], o[e]);
    }
  }

  if (qi < p.Sq) {
    // no keys at all: o = 0 (an empty P.V); a row that sees no key: 0 * inf = NaN, the reference's softmax of -inf
    const float inv = p.Sk == 0 ? 0.f : 1.0f / l;
    float* op = static_cast<float*>(p.o) + b * p.o_sb + (int64_t)qi * p.o_ss + h * p.o_sh + qd * DQ;
#pragma unroll
    for (int e = 0; e < DQ; e += 4) {
      const f32x4 v = {o[e] * inv, o[e + 1] * inv, o[e + 2] * inv, o[e + 3] * inv};
      *reinterpret_cast<f32x4*>(op + e) = v;
    }
    if (p.lse != nullptr && qd == 0) {
      const float lse = m == -INFINITY ? -INFINITY : m + logf(l);
      p.lse[(int64_t)bh * p.Sq + qi] = p.lse_base2 ? lse * kLog2e : lse;
    }
  }
}

template <int D, bool SOFTCAP, int EPI>
__global__ void __launch_bounds__(kThr) attn_col_f32_kernel(AttnParams p) {
  constexpr int DQ = D / 4;
  __shared__ __attribute__((aligned(16))) float Qs[kTile][D + 4];
  __shared__ float Ls[kTile];
  int kt, bh;
  map_block(p.n_tiles, p.B * p.Hq, false, kt, bh);
  const int b = bh / p.Hq, h = bh - b * p.Hq, hk = h / p.group;
  const int col = threadIdx.x >> 2, qd = threadIdx.x & 3;
  const int k0 = kt * kRows, kj = k0 + col;
  const float* qp = static_cast<const float*>(p.q) + b * p.q_sb + h * p.q_sh;
  const float* kp = static_cast<const float*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const float* lsep = p.lse + (int64_t)bh * p.Sq;

  float kv[DQ];
  const float* krow = kp + (int64_t)min(kj, p.Sk - 1) * p.k_ss + qd * DQ;
#pragma unroll
  for (int e = 0; e < DQ; e += 4) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(krow + e);
    kv[e] = v[0];
    kv[e + 1] = v[1];
    kv[e + 2] = v[2];
    kv[e + 3] = v[3];
  }

  // Query rows that can see any key of this workgroup.
  const int k_last = min(k0 + kRows, p.Sk) - 1;
  int q_begin = 0, q_end = p.Sq;
  if (p.causal) q_begin = max(0, k0 - p.offset);
  if (p.window > 0) q_end = min(p.Sq, k_last - p.offset + p.window);

  float sum = 0.f, sum2 = 0.f;
  int any = 0;
  for (int qb = (q_begin / kTile) * kTile; qb < q_end; qb += kTile) {
    __syncthreads();
    stage_rows<D>(Qs, qp, p.q_ss, qb, p.Sq);
    if (threadIdx.x < kTile) {
      const int qg = qb + threadIdx.x;
      Ls[threadIdx.x] = qg < p.Sq ? (p.lse_base2 ? lsep[qg] * kLn2 : lsep[qg]) : INFINITY;
    }
    __syncthreads();
#pragma unroll 4
    for (int i = 0; i < kTile; ++i) {
      const int qg = qb + i;
      const float x = f32_score<SOFTCAP>(quad_dot<D>(kv, &Qs[i][qd * DQ]), p);
      bool ok = qg < p.Sq && kj < p.Sk;
      if (p.causal) ok = ok && kj <= qg + p.offset;
      if (p.window > 0) ok = ok && qg + p.offset - kj < p.window;
      const float pe = ok ? expf(x - Ls[i]) : 0.f;
      if constexpr (EPI == kColAnyGe) {
        if (ok) any |= pe >= p.thr[(int64_t)qg * p.thr_rs + kj];  // masked pairs: corm_masked_or_kernel
      } else {
        sum += pe;
        if constexpr (EPI == kColSumSq) sum2 = fmaf(pe, pe, sum2);
      }
    }
  }
  if (qd == 0 && kj < p.Sk) {
    const int64_t idx = (int64_t)bh * p.Sk + kj;
    if constexpr (EPI == kColAnyGe) {
      p.any_out[idx] = (uint8_t)(any != 0);
    } else {
      p.colsum[idx] = sum;
      if constexpr (EPI == kColSumSq) p.colsum2[idx] = sum2;
    }
  }
}

template <int D, bool SOFTCAP>
void launch_fwd_f32_d(const AttnParams& p, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  hipLaunchKernelGGL((attn_fwd_f32_kernel<D, SOFTCAP>), dim3(grid), dim3(kThr), 0, st, p);
}
template <int D, bool SOFTCAP, int EPI>
void launch_col_f32_d(const AttnParams& p, hipStream_t st) {
  const unsigned grid = (unsigned)p.n_tiles * p.B * p.Hq;
  hipLaunchKernelGGL((attn_col_f32_kernel<D, SOFTCAP, EPI>), dim3(grid), dim3(kThr), 0, st, p);
}
template <int D>
void fwd_f32(const AttnParams& p, hipStream_t st) {
  if (p.softcap > 0.f) launch_fwd_f32_d<D, true>(p, st);
  else launch_fwd_f32_d<D, false>(p, st);
}
template <int D>
void col_f32(const AttnParams& p, int epi, hipStream_t st) {
  if (epi == kColSumSq) return launch_col_f32_d<D, false, kColSumSq>(p, st);
  if (epi == kColAnyGe) return launch_col_f32_d<D, false, kColAnyGe>(p, st);
  if (p.softcap > 0.f) launch_col_f32_d<D, true, kColSum>(p, st);
  else launch_col_f32_d<D, false, kColSum>(p, st);
}

}  // namespace

int f32_rows_per_tile() { return kRows; }

void launch_attn_f32_fwd(const AttnParams& p, int D, hipStream_t st) {
  if (D == 64) fwd_f32<64>(p, st);
  else if (D == 128) fwd_f32<128>(p, st);
  else fwd_f32<256>(p, st);
}

void launch_attn_f32_col(const AttnParams& p, int D, int epi, hipStream_t st) {
  if (D == 64) col_f32<64>(p, epi, st);
  else if (D == 128) col_f32<128>(p, epi, st);
  else col_f32<256>(p, epi, st);
}

}  // namespace dgg_attn
