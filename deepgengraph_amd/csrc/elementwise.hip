// Elementwise kernels of the Llama layer around attention: RMSNorm, fused residual-add + RMSNorm,
// SiLU-and-mul and online rotary embedding. All are HBM-bound: 16-byte vector loads/stores, one pass
// over the data (the row of an RMSNorm is held in registers between the reduction and the scaling),
// fp32 arithmetic, and rounding to the storage type at the points where the reference rounds.
#include <algorithm>

#include "common.h"

namespace {

// Vector traits: a 16-byte chunk holds EPV elements.
template <typename T>
struct VecOf;
template <>
struct VecOf<F16> {
  typedef f16x8 type;
  static constexpr int EPV = 8;
};
template <>
struct VecOf<BF16> {
  typedef bf16x8 type;
  static constexpr int EPV = 8;
};
template <>
struct VecOf<F32> {
  typedef f32x4 type;
  static constexpr int EPV = 4;
};

template <typename T>
__device__ __forceinline__ float round_t(float x) {
  return to_f<typename T::scalar>(to_s<typename T::scalar>(x));
}
template <>
__device__ __forceinline__ float round_t<F32>(float x) {
  return x;
}

// Block-wide sum for up to 1024 threads (wave64 shuffles, then one LDS hop).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = (blockDim.x + 63) >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = lane < nw ? red[lane] : 0.f;
  t = wave_sum(t);
  return t;
}

// ---------------------------------------------------------------------------------------------
// RMSNorm (csrc/norm.cu:34-56). Vector path: the row is read once into registers (NV chunks per thread),
// together with the matching weight chunks. The row and the output use non-temporal accesses (each is touched
// once): 4096 x 4096 bf16 in 9.9-10.4 us against 12.4 us with ordinary ones. The weight, read by every row, and
// the residual of the fused form keep ordinary accesses.
// RESID: fused residual add (csrc/norm.cu:59-83): v = in + res; res = T(v); variance from the unrounded v;
// output from the rounded residual.
// ---------------------------------------------------------------------------------------------
template <typename T, int NV, bool RESID>
__device__ __forceinline__ void rms_row_vec(int64_t row, typename T::scalar* __restrict__ out,
                                            const typename T::scalar* __restrict__ in,
                                            typename T::scalar* __restrict__ res,
                                            const typename T::scalar* __restrict__ w, int hidden, int64_t in_rs,
                                            int64_t out_rs, int64_t res_rs, float eps, float* red) {
  typedef typename VecOf<T>::type V;
  constexpr int EPV = VecOf<T>::EPV;
  const int nvec = hidden / EPV;
  const typename T::scalar* x = in + row * in_rs;
  float vals[NV][EPV];
  V wv[NV];  // the weight slice, loaded with the row so that its latency is not paid after the reduction
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * blockDim.x;
    if (c < nvec) {
      V a = ld16_nt<V>(x + (int64_t)c * EPV);
      wv[i] = ld16<V>(w + (int64_t)c * EPV);
      if constexpr (RESID) {
        typename T::scalar* r = res + row * res_rs + (int64_t)c * EPV;
        V b = ld16<V>(r);
        V rr;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          float v = to_f(a[e]) + to_f(b[e]);
          ss += v * v;
          rr[e] = to_s<typename T::scalar>(v);
          vals[i][e] = to_f(rr[e]);
        }
        st16<V>(r, rr);
      } else {
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          float v = to_f(a[e]);
          vals[i][e] = v;
          ss += v * v;
        }
      }
    }
  }
  ss = block_sum(ss, red);
  const float s = rsqrtf(ss / (float)hidden + eps);
  typename T::scalar* y = out + row * out_rs;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * blockDim.x;
    if (c < nvec) {
      V o;
#pragma unroll
      for (int e = 0; e < EPV; ++e) o[e] = to_s<typename T::scalar>(round_t<T>(vals[i][e] * s) * to_f(wv[i][e]));
      st16_nt<V>(y + (int64_t)c * EPV, o);
    }
  }
}

template <typename T, int NV, bool RESID>
__global__ void __launch_bounds__(1024) rms_norm_vec_kernel(typename T::scalar* __restrict__ out,
                                                             const typename T::scalar* __restrict__ in,
                                                             typename T::scalar* __restrict__ res,
                                                             const typename T::scalar* __restrict__ w,
                                                             int hidden, int64_t in_rs, int64_t out_rs,
                                                             int64_t res_rs, float eps) {
  __shared__ float red[16];
  rms_row_vec<T, NV, RESID>(blockIdx.x, out, in, res, w, hidden, in_rs, out_rs, res_rs, eps, red);
}

// Scalar fallback for any hidden size / alignment: two passes over the row (second pass re-reads it).
template <typename T, bool RESID>
__global__ void __launch_bounds__(1024) rms_norm_scalar_kernel(typename T::scalar* __restrict__ out,
                                                                const typename T::scalar* __restrict__ in,
                                                                typename T::scalar* __restrict__ res,
                                                                const typename T::scalar* __restrict__ w,
                                                                int hidden, int64_t in_rs, int64_t out_rs,
                                                                int64_t res_rs, float eps) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    float v = to_f(in[row * in_rs + i]);
    if constexpr (RESID) {
      v += to_f(res[row * res_rs + i]);
      res[row * res_rs + i] = to_s<typename T::scalar>(v);
    }
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float s = rsqrtf(ss / (float)hidden + eps);
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    float v = RESID ? to_f(res[row * res_rs + i]) : to_f(in[row * in_rs + i]);
    out[row * out_rs + i] = to_s<typename T::scalar>(round_t<T>(v * s) * to_f(w[i]));
  }
}

// ---------------------------------------------------------------------------------------------
// SiLU-and-mul (csrc/activation.cu:6-22): out = T(T(silu(g)) * u), silu in fp32.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float silu_f(float g) { return g * fast_rcp(1.f + fast_exp2(-g * kLog2e)); }

// Vector SiLU-and-mul over the 16-byte chunks t = blk * blockDim + tid, stepping by nblk * blockDim. Non-temporal
// loads and stores (every element is touched once): 4096 x 11008 bf16 in 40.4-41.0 against 41.2-41.8 us.
template <typename T>
__device__ __forceinline__ void silu_vec_range(typename T::scalar* __restrict__ out,
                                               const typename T::scalar* __restrict__ in, int64_t rows, int64_t d,
                                               int64_t in_rs, int64_t out_rs, int64_t blk, int64_t nblk) {
  typedef typename VecOf<T>::type V;
  constexpr int EPV = VecOf<T>::EPV;
  const int64_t vpr = d / EPV;
  const int64_t total = rows * vpr;
  for (int64_t t = blk * blockDim.x + threadIdx.x; t < total; t += nblk * blockDim.x) {
    const int64_t r = t / vpr, c = (t - r * vpr) * EPV;
    const typename T::scalar* src = in + r * in_rs;
    V g = ld16_nt<V>(src + c);
    V u = ld16_nt<V>(src + d + c);
    V o;
#pragma unroll
    for (int e = 0; e < EPV; ++e) o[e] = to_s<typename T::scalar>(round_t<T>(silu_f(to_f(g[e]))) * to_f(u[e]));
    st16_nt<V>(out + r * out_rs + c, o);
  }
}

template <typename T>
__global__ void __launch_bounds__(256) silu_and_mul_vec_kernel(typename T::scalar* __restrict__ out,
                                                                const typename T::scalar* __restrict__ in,
                                                                int64_t rows, int64_t d, int64_t in_rs,
                                                                int64_t out_rs) {
  silu_vec_range<T>(out, in, rows, d, in_rs, out_rs, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------------------------------------
// RMSNorm and SiLU-and-mul in one launch (the decode pre-step: a few rows of each, where each op alone is a few
// microseconds of launch ramp): workgroups 0 .. norm_rows-1 normalise one row each, the others split the SiLU
// chunks between them.
// ---------------------------------------------------------------------------------------------
template <typename T, int NV>
__global__ void __launch_bounds__(1024) rms_silu_kernel(typename T::scalar* __restrict__ norm_out,
                                                         const typename T::scalar* __restrict__ norm_in,
                                                         const typename T::scalar* __restrict__ w, int hidden,
                                                         int64_t norm_in_rs, int64_t norm_out_rs, float eps,
                                                         int norm_rows, typename T::scalar* __restrict__ act_out,
                                                         const typename T::scalar* __restrict__ act_in,
                                                         int64_t act_rows, int64_t d, int64_t act_in_rs,
                                                         int64_t act_out_rs) {
  __shared__ float red[16];
  if ((int)blockIdx.x < norm_rows)
    rms_row_vec<T, NV, false>(blockIdx.x, norm_out, norm_in, nullptr, w, hidden, norm_in_rs, norm_out_rs, 0, eps,
                              red);
  else
    silu_vec_range<T>(act_out, act_in, act_rows, d, act_in_rs, act_out_rs, blockIdx.x - norm_rows,
                      gridDim.x - norm_rows);
}

template <typename T>
__global__ void __launch_bounds__(256) silu_and_mul_scalar_kernel(typename T::scalar* __restrict__ out,
                                                                   const typename T::scalar* __restrict__ in,
                                                                   int64_t rows, int64_t d, int64_t in_rs,
                                                                   int64_t out_rs) {
  const int64_t total = rows * d;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / d, c = t - r * d;
    float g = to_f(in[r * in_rs + c]);
    float u = to_f(in[r * in_rs + d + c]);
    out[r * out_rs + c] = to_s<typename T::scalar>(round_t<T>(silu_f(g)) * u);
  }
}

// ---------------------------------------------------------------------------------------------
// Online rotary (csrc/pos_encoding.cu:64-113). One workgroup per token: the D/2 (cos, sin) pairs are
// computed once into LDS with accurate powf / sincosf (angles reach thousands of radians), then every
// (head, 8-pair group) of q and k is rotated with 16-byte loads, the first two per thread issued before the
// angles are computed. VEC=false: scalar element path.
// ---------------------------------------------------------------------------------------------
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) rotary_online_kernel(const int32_t* __restrict__ pos,
                                                             typename T::scalar* __restrict__ q,
                                                             typename T::scalar* __restrict__ k, int hq,
                                                             int hk, int D, int64_t q_rs, int64_t k_rs,
                                                             float theta) {
  __shared__ float cs[256], sn[256];
  typedef typename T::scalar S;
  const int half = D / 2;
  const int64_t tok = blockIdx.x;
  const float p = (float)pos[tok];
  auto angles = [&]() {
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      const float ang = p / powf(theta, (float)(2 * i) / (float)D);
      float s, c;
      sincosf(ang, &s, &c);
      cs[i] = c;
      sn[i] = s;
    }
  };
  if constexpr (VEC) {
    typedef typename VecOf<T>::type V;
    constexpr int EPV = VecOf<T>::EPV;
    // Items (head, 8-pair group) of this thread whose loads are issued before the angles are computed, so that
    // the memory latency and the powf / sincosf latency overlap (two per thread at 32 + 32 heads of 128).
    constexpr int PF = 2;
    const int gph = half / EPV;  // pair groups per head
    const int items = (hq + hk) * gph;
    auto item_base = [&](int it, int& i0) -> S* {
      const int h = it / gph, gi = it - h * gph;
      i0 = gi * EPV;
      return h < hq ? q + tok * q_rs + (int64_t)h * D : k + tok * k_rs + (int64_t)(h - hq) * D;
    };
    auto rotate = [&](S* base, int i0, const V& x, const V& y) {
      V xo, yo;
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float c = cs[i0 + e], s = sn[i0 + e];
        const float xf = to_f(x[e]), yf = to_f(y[e]);
        xo[e] = to_s<S>(xf * c - yf * s);
        yo[e] = to_s<S>(yf * c + xf * s);
      }
      st16<V>(base + i0, xo);
      st16<V>(base + half + i0, yo);
    };
    V px[PF], py[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int it = threadIdx.x + j * blockDim.x;
      if (it < items) {
        int i0;
        const S* base = item_base(it, i0);
        px[j] = ld16<V>(base + i0);
        py[j] = ld16<V>(base + half + i0);
      }
    }
    angles();
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int it = threadIdx.x + j * blockDim.x;
      if (it < items) {
        int i0;
        S* base = item_base(it, i0);
        rotate(base, i0, px[j], py[j]);
      }
    }
    for (int it = threadIdx.x + PF * blockDim.x; it < items; it += blockDim.x) {
      int i0;
      S* base = item_base(it, i0);
      rotate(base, i0, ld16<V>(base + i0), ld16<V>(base + half + i0));
    }
  } else {
    angles();
    __syncthreads();
    const int items = (hq + hk) * half;
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
      const int h = it / half, i = it - h * half;
      S* base = h < hq ? q + tok * q_rs + (int64_t)h * D : k + tok * k_rs + (int64_t)(h - hq) * D;
      const float xf = to_f(base[i]), yf = to_f(base[half + i]);
      const float c = cs[i], s = sn[i];
      base[i] = to_s<S>(xf * c - yf * s);
      base[half + i] = to_s<S>(yf * c + xf * s);
    }
  }
}

template <typename T, int NV, bool RESID>
void launch_rms_vec(int threads, void* out, const void* in, void* res, const void* w, int64_t rows, int hidden,
                    int64_t in_rs, int64_t out_rs, int64_t res_rs, float eps, hipStream_t st) {
  typedef typename T::scalar S;
  hipLaunchKernelGGL((rms_norm_vec_kernel<T, NV, RESID>), dim3((unsigned)rows), dim3(threads), 0, st, (S*)out,
                     (const S*)in, (S*)res, (const S*)w, hidden, in_rs, out_rs, res_rs, eps);
}

template <typename T, bool RESID>
int rms_dispatch(void* out, const void* in, void* res, const void* w, int64_t rows, int64_t hidden, int64_t in_rs,
                 int64_t out_rs, int64_t res_rs, float eps, hipStream_t st) {
  typedef typename T::scalar S;
  constexpr int EPV = VecOf<T>::EPV;
  const bool vec = hidden % EPV == 0 && in_rs % EPV == 0 && out_rs % EPV == 0 && (!RESID || res_rs % EPV == 0) &&
                   dgg::aligned16(out) && dgg::aligned16(in) && dgg::aligned16(w) && (!RESID || dgg::aligned16(res));
  const int64_t nvec = hidden / EPV;
  if (vec && nvec <= 8 * 1024) {
    // With enough rows to fill the chip (>= 1024 workgroups), about four 16-byte chunks per thread (measured at
    // 4096 x 4096 bf16: 128 threads x 4 chunks 11.4 us, 256 x 2 11.9 us, 512 x 1 12.5 us; a plain copy of the same
    // bytes 10.1-10.7 us); with few rows, one chunk per thread, so each row's loads are spread over more threads
    // (64 x 4096 fp16: 2.85 us vs 3.57 us at four chunks). Up to 8 chunks for rows over 4096 chunks (1024 threads).
    const int64_t per_thread = rows >= 1024 ? 4 : 1;
    int threads = (int)(((nvec + per_thread - 1) / per_thread + 63) / 64 * 64);
    if (threads > 1024) threads = 1024;  // then at most 8 chunks per thread, as nvec <= 8192
    const int64_t nv = (nvec + threads - 1) / threads;
    if (nv <= 1) launch_rms_vec<T, 1, RESID>(threads, out, in, res, w, rows, (int)hidden, in_rs, out_rs, res_rs, eps, st);
    else if (nv <= 2) launch_rms_vec<T, 2, RESID>(threads, out, in, res, w, rows, (int)hidden, in_rs, out_rs, res_rs, eps, st);
    else if (nv <= 4) launch_rms_vec<T, 4, RESID>(threads, out, in, res, w, rows, (int)hidden, in_rs, out_rs, res_rs, eps, st);
    else launch_rms_vec<T, 8, RESID>(threads, out, in, res, w, rows, (int)hidden, in_rs, out_rs, res_rs, eps, st);
  } else {
    const int threads = hidden >= 1024 ? 1024 : (int)((hidden + 63) / 64 * 64);
    hipLaunchKernelGGL((rms_norm_scalar_kernel<T, RESID>), dim3((unsigned)rows), dim3(threads), 0, st, (S*)out,
                       (const S*)in, (S*)res, (const S*)w, (int)hidden, in_rs, out_rs, res_rs, eps);
  }
  return dgg::check_launch(RESID ? "fused_add_rms_norm" : "rms_norm");
}

template <typename T>
int silu_dispatch(void* out, const void* in, int64_t rows, int64_t d, int64_t in_rs, int64_t out_rs, hipStream_t st) {
  typedef typename T::scalar S;
  constexpr int EPV = VecOf<T>::EPV;
  const bool vec = d % EPV == 0 && in_rs % EPV == 0 && out_rs % EPV == 0 && dgg::aligned16(out) && dgg::aligned16(in);
  const int64_t work = vec ? rows * (d / EPV) : rows * d;
  int64_t blocks = (work + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;
  if (vec)
    hipLaunchKernelGGL((silu_and_mul_vec_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, st, (S*)out, (const S*)in,
                       rows, d, in_rs, out_rs);
  else
    hipLaunchKernelGGL((silu_and_mul_scalar_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, st, (S*)out,
                       (const S*)in, rows, d, in_rs, out_rs);
  return dgg::check_launch("silu_and_mul");
}

// ---------------------------------------------------------------------------------------------
// Rotary with a (cos, sin) cache (csrc/pos_encoding.cu:7-61, host 152-178): row pos of the cache is
// [cos (rot_dim/2) | sin (rot_dim/2)] in the storage type. NEOX pairs (i, i + rot_dim/2), GPT-J pairs (2i, 2i + 1),
// i < rot_dim/2; the head dims past rot_dim are left as they are. The reference computes in its scalar_t: for the
// 16-bit types each product and then the difference / sum is rounded to the storage type (c10 Half / BFloat16
// operators compute in float and round), fp32 is plain fp32 arithmetic. One workgroup per token; VEC: 16-byte
// chunks (NeoX: 8 pairs per item, GPT-J: 4 pairs), else one pair per item. A token whose position lies outside
// [0, max_position) is left unchanged (nothing is read outside the cache).
// ---------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void rot_pair(float x, float y, float c, float s, float& xo, float& yo) {
#pragma clang fp contract(off)
  xo = round_t<T>(round_t<T>(x * c) - round_t<T>(y * s));
  yo = round_t<T>(round_t<T>(y * c) + round_t<T>(x * s));
}

template <typename T, bool NEOX, bool VEC>
__global__ void __launch_bounds__(256) rotary_cache_kernel(const int32_t* __restrict__ pos,
                                                            typename T::scalar* __restrict__ q,
                                                            typename T::scalar* __restrict__ k,
                                                            const typename T::scalar* __restrict__ cache, int hq,
                                                            int hk, int head_size, int rot_dim, int64_t max_pos,
                                                            int64_t q_rs, int64_t k_rs) {
  typedef typename T::scalar S;
  const int64_t tok = blockIdx.x;
  const int64_t p = pos[tok];
  if (p < 0 || p >= max_pos) return;
  const int embed = rot_dim / 2;
  const S* cr = cache + p * rot_dim;  // cos at cr[i], sin at cr[embed + i]
  auto head_base = [&](int h) -> S* {
    return h < hq ? q + tok * q_rs + (int64_t)h * head_size : k + tok * k_rs + (int64_t)(h - hq) * head_size;
  };
  if constexpr (VEC) {
    typedef typename VecOf<T>::type V;
    constexpr int EPV = VecOf<T>::EPV;
    if constexpr (NEOX) {
      const int per_head = embed / EPV;  // 8-pair groups
      const int items = (hq + hk) * per_head;
      for (int it = threadIdx.x; it < items; it += blockDim.x) {
        const int h = it / per_head, i0 = (it - h * per_head) * EPV;
        S* base = head_base(h);
        const V x = ld16<V>(base + i0), y = ld16<V>(base + embed + i0);
        const V c = ld16<V>(cr + i0), sn = ld16<V>(cr + embed + i0);
        V xo, yo;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          float a, b;
          rot_pair<T>(to_f(x[e]), to_f(y[e]), to_f(c[e]), to_f(sn[e]), a, b);
          xo[e] = to_s<S>(a);
          yo[e] = to_s<S>(b);
        }
        st16<V>(base + i0, xo);
        st16<V>(base + embed + i0, yo);
      }
    } else {
      constexpr int PPC = EPV / 2;       // pairs per 16-byte chunk
      const int per_head = rot_dim / EPV;  // chunks
      const int items = (hq + hk) * per_head;
      for (int it = threadIdx.x; it < items; it += blockDim.x) {
        const int h = it / per_head, j = it - h * per_head;
        S* base = head_base(h) + j * EPV;
        const V xy = ld16<V>(base);
        V o;
#pragma unroll
        for (int e = 0; e < PPC; ++e) {
          float a, b;
          const int r = j * PPC + e;
          rot_pair<T>(to_f(xy[2 * e]), to_f(xy[2 * e + 1]), to_f(cr[r]), to_f(cr[embed + r]), a, b);
          o[2 * e] = to_s<S>(a);
          o[2 * e + 1] = to_s<S>(b);
        }
        st16<V>(base, o);
      }
    }
  } else {
    const int items = (hq + hk) * embed;
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
      const int h = it / embed, r = it - h * embed;
      S* base = head_base(h);
      const int xi = NEOX ? r : 2 * r, yi = NEOX ? embed + r : 2 * r + 1;
      float a, b;
      rot_pair<T>(to_f(base[xi]), to_f(base[yi]), to_f(cr[r]), to_f(cr[embed + r]), a, b);
      base[xi] = to_s<S>(a);
      base[yi] = to_s<S>(b);
    }
  }
}

template <typename T>
int rotary_cache_dispatch(const int32_t* pos, void* q, void* k, const void* cache, int64_t tokens, int64_t hq,
                          int64_t hk, int64_t hs, int64_t rot_dim, int64_t max_pos, int64_t q_rs, int64_t k_rs,
                          bool neox, hipStream_t st) {
  typedef typename T::scalar S;
  constexpr int EPV = VecOf<T>::EPV;
  const bool vec = (neox ? (rot_dim / 2) % EPV == 0 : rot_dim % EPV == 0) && hs % EPV == 0 && q_rs % EPV == 0 &&
                   (k == nullptr || k_rs % EPV == 0) && dgg::aligned16(q) && (k == nullptr || dgg::aligned16(k)) &&
                   dgg::aligned16(cache) && rot_dim % EPV == 0;
  const int64_t items = (hq + hk) * (vec ? (neox ? rot_dim / 2 / EPV : rot_dim / EPV) : rot_dim / 2);
  int threads = (int)((items + 63) / 64 * 64);
  threads = std::max(64, std::min(256, threads));
  const dim3 grid((unsigned)tokens), block(threads);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, st, pos, (S*)q, (S*)k, (const S*)cache, (int)hq, (int)hk, (int)hs,
                       (int)rot_dim, max_pos, q_rs, k_rs);
  };
  if (neox) vec ? args(rotary_cache_kernel<T, true, true>) : args(rotary_cache_kernel<T, true, false>);
  else vec ? args(rotary_cache_kernel<T, false, true>) : args(rotary_cache_kernel<T, false, false>);
  return dgg::check_launch("rotary_embedding");
}

template <typename T, int NV>
void launch_rms_silu(int threads, unsigned silu_blocks, void* norm_out, const void* norm_in, const void* w,
                     int64_t norm_rows, int hidden, int64_t n_in_rs, int64_t n_out_rs, float eps, void* act_out,
                     const void* act_in, int64_t act_rows, int64_t d, int64_t a_in_rs, int64_t a_out_rs,
                     hipStream_t st) {
  typedef typename T::scalar S;
  hipLaunchKernelGGL((rms_silu_kernel<T, NV>), dim3((unsigned)norm_rows + silu_blocks), dim3(threads), 0, st,
                     (S*)norm_out, (const S*)norm_in, (const S*)w, hidden, n_in_rs, n_out_rs, eps, (int)norm_rows,
                     (S*)act_out, (const S*)act_in, act_rows, d, a_in_rs, a_out_rs);
}

// One launch when both ops take the vector path and the norm rows fit one workgroup each; otherwise the two
// kernels one after the other.
template <typename T>
int rms_silu_dispatch(void* norm_out, const void* norm_in, const void* w, int64_t norm_rows, int64_t hidden,
                      int64_t n_in_rs, int64_t n_out_rs, float eps, void* act_out, const void* act_in, int64_t act_rows,
                      int64_t d, int64_t a_in_rs, int64_t a_out_rs, hipStream_t st) {
  constexpr int EPV = VecOf<T>::EPV;
  const bool vec = hidden % EPV == 0 && n_in_rs % EPV == 0 && n_out_rs % EPV == 0 && dgg::aligned16(norm_out) &&
                   dgg::aligned16(norm_in) && dgg::aligned16(w) && d % EPV == 0 && a_in_rs % EPV == 0 &&
                   a_out_rs % EPV == 0 && dgg::aligned16(act_out) && dgg::aligned16(act_in);
  const int64_t nvec = hidden / EPV;
  if (!vec || nvec > 8 * 1024 || norm_rows == 0 || act_rows == 0 || norm_rows > (1 << 20)) {
    if (norm_rows > 0)
      if (int rc = rms_dispatch<T, false>(norm_out, norm_in, nullptr, w, norm_rows, hidden, n_in_rs, n_out_rs, 0, eps,
                                          st))
        return rc;
    if (act_rows > 0) return silu_dispatch<T>(act_out, act_in, act_rows, d, a_in_rs, a_out_rs, st);
    return DGG_OK;
  }
  // one 16-byte chunk of the norm row per thread (as the few-row RMSNorm launch), up to 8 for wide rows
  int threads = (int)((nvec + 63) / 64 * 64);
  if (threads > 1024) threads = 1024;
  const int64_t nv = (nvec + threads - 1) / threads;
  const int64_t silu_vecs = act_rows * (d / EPV);
  const unsigned silu_blocks = (unsigned)std::min<int64_t>(256 * 64, (silu_vecs + threads - 1) / threads);
  const int h = (int)hidden;
  if (nv <= 1)
    launch_rms_silu<T, 1>(threads, silu_blocks, norm_out, norm_in, w, norm_rows, h, n_in_rs, n_out_rs, eps, act_out,
                          act_in, act_rows, d, a_in_rs, a_out_rs, st);
  else if (nv <= 2)
    launch_rms_silu<T, 2>(threads, silu_blocks, norm_out, norm_in, w, norm_rows, h, n_in_rs, n_out_rs, eps, act_out,
                          act_in, act_rows, d, a_in_rs, a_out_rs, st);
  else if (nv <= 4)
    launch_rms_silu<T, 4>(threads, silu_blocks, norm_out, norm_in, w, norm_rows, h, n_in_rs, n_out_rs, eps, act_out,
                          act_in, act_rows, d, a_in_rs, a_out_rs, st);
  else
    launch_rms_silu<T, 8>(threads, silu_blocks, norm_out, norm_in, w, norm_rows, h, n_in_rs, n_out_rs, eps, act_out,
                          act_in, act_rows, d, a_in_rs, a_out_rs, st);
  return dgg::check_launch("rms_norm_silu_and_mul");
}

template <typename T>
int rotary_dispatch(const int32_t* pos, void* q, void* k, int64_t tokens, int64_t hq, int64_t hk, int64_t D,
                    int64_t q_rs, int64_t k_rs, float theta, hipStream_t st) {
  typedef typename T::scalar S;
  constexpr int EPV = VecOf<T>::EPV;
  const bool vec = (D / 2) % EPV == 0 && q_rs % EPV == 0 && (k == nullptr || k_rs % EPV == 0) && dgg::aligned16(q) &&
                   (k == nullptr || dgg::aligned16(k));
  const int64_t items = (hq + hk) * (vec ? D / 2 / EPV : D / 2);
  int threads = (int)((items + 63) / 64 * 64);
  if (threads > 256) threads = 256;
  if (threads < 64) threads = 64;
  if (vec)
    hipLaunchKernelGGL((rotary_online_kernel<T, true>), dim3((unsigned)tokens), dim3(threads), 0, st, pos, (S*)q,
                       (S*)k, (int)hq, (int)hk, (int)D, q_rs, k_rs, theta);
  else
    hipLaunchKernelGGL((rotary_online_kernel<T, false>), dim3((unsigned)tokens), dim3(threads), 0, st, pos, (S*)q,
                       (S*)k, (int)hq, (int)hk, (int)D, q_rs, k_rs, theta);
  return dgg::check_launch("rotary_embedding_online");
}

int check_rows(const char* op, int64_t rows, int64_t cols, int64_t in_rs, int64_t out_rs, int64_t min_in_rs) {
  DGG_REQUIRE(rows >= 0, DGG_ERR_SHAPE, "%s: rows must be >= 0 (got %lld)", op, (long long)rows);
  DGG_REQUIRE(rows <= 0x7fffffff, DGG_ERR_SHAPE, "%s: rows must be < 2^31 (got %lld)", op, (long long)rows);
  DGG_REQUIRE(cols > 0, DGG_ERR_SHAPE, "%s: row width must be > 0 (got %lld)", op, (long long)cols);
  DGG_REQUIRE(cols <= 0x7fffffff, DGG_ERR_SHAPE, "%s: row width must be < 2^31 (got %lld)", op, (long long)cols);
  DGG_REQUIRE(in_rs >= min_in_rs, DGG_ERR_STRIDE, "%s: input row stride %lld is smaller than the row (%lld)", op,
              (long long)in_rs, (long long)min_in_rs);
  DGG_REQUIRE(out_rs >= cols, DGG_ERR_STRIDE, "%s: output row stride %lld is smaller than the row (%lld)", op,
              (long long)out_rs, (long long)cols);
  return DGG_OK;
}

}  // namespace

extern "C" int dgg_rms_norm(void* out, const void* input, const void* weight, int64_t rows, int64_t hidden,
                            int64_t in_row_stride, int64_t out_row_stride, int dtype, float epsilon, void* stream) {
  DGG_REQUIRE(dgg::valid_dtype(dtype), DGG_ERR_DTYPE, "rms_norm: unsupported dtype code %d", dtype);
  if (int rc = check_rows("rms_norm", rows, hidden, in_row_stride, out_row_stride, hidden)) return rc;
  if (rows == 0) return DGG_OK;
  DGG_REQUIRE(out && input && weight, DGG_ERR_NULL, "rms_norm: null pointer");
  hipStream_t st = dgg::as_stream(stream);
  switch (dtype) {
    case DGG_F16: return rms_dispatch<F16, false>(out, input, nullptr, weight, rows, hidden, in_row_stride, out_row_stride, 0, epsilon, st);
    case DGG_BF16: return rms_dispatch<BF16, false>(out, input, nullptr, weight, rows, hidden, in_row_stride, out_row_stride, 0, epsilon, st);
    default: return rms_dispatch<F32, false>(out, input, nullptr, weight, rows, hidden, in_row_stride, out_row_stride, 0, epsilon, st);
  }
}

extern "C" int dgg_fused_add_rms_norm(void* input, void* residual, const void* weight, int64_t rows, int64_t hidden,
                                      int64_t in_row_stride, int64_t res_row_stride, int dtype, float epsilon,
                                      void* stream) {
  DGG_REQUIRE(dgg::valid_dtype(dtype), DGG_ERR_DTYPE, "fused_add_rms_norm: unsupported dtype code %d", dtype);
  if (int rc = check_rows("fused_add_rms_norm", rows, hidden, in_row_stride, in_row_stride, hidden)) return rc;
  DGG_REQUIRE(res_row_stride >= hidden, DGG_ERR_STRIDE, "fused_add_rms_norm: residual row stride %lld < hidden %lld",
              (long long)res_row_stride, (long long)hidden);
  if (rows == 0) return DGG_OK;
  DGG_REQUIRE(input && residual && weight, DGG_ERR_NULL, "fused_add_rms_norm: null pointer");
  hipStream_t st = dgg::as_stream(stream);
  switch (dtype) {
    case DGG_F16: return rms_dispatch<F16, true>(input, input, residual, weight, rows, hidden, in_row_stride, in_row_stride, res_row_stride, epsilon, st);
    case DGG_BF16: return rms_dispatch<BF16, true>(input, input, residual, weight, rows, hidden, in_row_stride, in_row_stride, res_row_stride, epsilon, st);
    default: return rms_dispatch<F32, true>(input, input, residual, weight, rows, hidden, in_row_stride, in_row_stride, res_row_stride, epsilon, st);
  }
}

extern "C" int dgg_silu_and_mul(void* out, const void* input, int64_t rows, int64_t d, int64_t in_row_stride,
                                int64_t out_row_stride, int dtype, void* stream) {
  DGG_REQUIRE(dgg::valid_dtype(dtype), DGG_ERR_DTYPE, "silu_and_mul: unsupported dtype code %d", dtype);
  if (int rc = check_rows("silu_and_mul", rows, d, in_row_stride, out_row_stride, 2 * d)) return rc;
  if (rows == 0) return DGG_OK;
  DGG_REQUIRE(out && input, DGG_ERR_NULL, "silu_and_mul: null pointer");
  hipStream_t st = dgg::as_stream(stream);
  switch (dtype) {
    case DGG_F16: return silu_dispatch<F16>(out, input, rows, d, in_row_stride, out_row_stride, st);
    case DGG_BF16: return silu_dispatch<BF16>(out, input, rows, d, in_row_stride, out_row_stride, st);
    default: return silu_dispatch<F32>(out, input, rows, d, in_row_stride, out_row_stride, st);
  }
}

extern "C" int dgg_rotary_embedding(const int32_t* positions, void* query, void* key, int64_t tokens,
                                    int64_t head_num, int64_t kv_head_num, int64_t head_size, int64_t q_row_stride,
                                    int64_t k_row_stride, const void* cos_sin_cache, int64_t rot_dim,
                                    int64_t max_position, int is_neox, int dtype, void* stream) {
  DGG_REQUIRE(dgg::valid_dtype(dtype), DGG_ERR_DTYPE, "rotary_embedding: unsupported dtype code %d", dtype);
  DGG_REQUIRE(tokens >= 0 && tokens <= 0x7fffffff, DGG_ERR_SHAPE, "rotary_embedding: bad token count %lld",
              (long long)tokens);
  DGG_REQUIRE(head_size > 0 && head_num >= 0 && kv_head_num >= 0 && head_num + kv_head_num < (1 << 20),
              DGG_ERR_SHAPE, "rotary_embedding: bad head sizes");
  DGG_REQUIRE(rot_dim >= 2 && rot_dim % 2 == 0 && rot_dim <= head_size, DGG_ERR_SHAPE,
              "rotary_embedding: rot_dim %lld must be even and in [2, head_size = %lld]", (long long)rot_dim,
              (long long)head_size);
  DGG_REQUIRE(max_position >= 0, DGG_ERR_SHAPE, "rotary_embedding: max_position must be >= 0");
  DGG_REQUIRE(q_row_stride >= head_num * head_size && (key == nullptr || k_row_stride >= kv_head_num * head_size),
              DGG_ERR_STRIDE, "rotary_embedding: a row stride is smaller than the row");
  if (key == nullptr) kv_head_num = 0;
  if (tokens == 0 || head_num + kv_head_num == 0) return DGG_OK;
  DGG_REQUIRE(positions && query && cos_sin_cache, DGG_ERR_NULL, "rotary_embedding: null pointer");
  hipStream_t st = dgg::as_stream(stream);
  const bool neox = is_neox != 0;
  switch (dtype) {
    case DGG_F16:
      return rotary_cache_dispatch<F16>(positions, query, key, cos_sin_cache, tokens, head_num, kv_head_num, head_size,
                                        rot_dim, max_position, q_row_stride, k_row_stride, neox, st);
    case DGG_BF16:
      return rotary_cache_dispatch<BF16>(positions, query, key, cos_sin_cache, tokens, head_num, kv_head_num,
                                         head_size, rot_dim, max_position, q_row_stride, k_row_stride, neox, st);
    default:
      return rotary_cache_dispatch<F32>(positions, query, key, cos_sin_cache, tokens, head_num, kv_head_num, head_size,
                                        rot_dim, max_position, q_row_stride, k_row_stride, neox, st);
  }
}

extern "C" int dgg_rms_norm_silu_and_mul(void* norm_out, const void* norm_in, const void* weight, int64_t norm_rows,
                                         int64_t hidden, int64_t norm_in_row_stride, int64_t norm_out_row_stride,
                                         float epsilon, void* act_out, const void* act_in, int64_t act_rows, int64_t d,
                                         int64_t act_in_row_stride, int64_t act_out_row_stride, int dtype,
                                         void* stream) {
  DGG_REQUIRE(dgg::valid_dtype(dtype), DGG_ERR_DTYPE, "rms_norm_silu_and_mul: unsupported dtype code %d", dtype);
  if (int rc = check_rows("rms_norm_silu_and_mul", norm_rows, hidden, norm_in_row_stride, norm_out_row_stride, hidden))
    return rc;
  if (int rc = check_rows("rms_norm_silu_and_mul", act_rows, d, act_in_row_stride, act_out_row_stride, 2 * d)) return rc;
  if (norm_rows == 0 && act_rows == 0) return DGG_OK;
  DGG_REQUIRE((norm_rows == 0 || (norm_out && norm_in && weight)) && (act_rows == 0 || (act_out && act_in)),
              DGG_ERR_NULL, "rms_norm_silu_and_mul: null pointer");
  hipStream_t st = dgg::as_stream(stream);
  switch (dtype) {
    case DGG_F16:
      return rms_silu_dispatch<F16>(norm_out, norm_in, weight, norm_rows, hidden, norm_in_row_stride,
                                    norm_out_row_stride, epsilon, act_out, act_in, act_rows, d, act_in_row_stride,
                                    act_out_row_stride, st);
    case DGG_BF16:
      return rms_silu_dispatch<BF16>(norm_out, norm_in, weight, norm_rows, hidden, norm_in_row_stride,
                                     norm_out_row_stride, epsilon, act_out, act_in, act_rows, d, act_in_row_stride,
                                     act_out_row_stride, st);
    default:
      return rms_silu_dispatch<F32>(norm_out, norm_in, weight, norm_rows, hidden, norm_in_row_stride,
                                    norm_out_row_stride, epsilon, act_out, act_in, act_rows, d, act_in_row_stride,
                                    act_out_row_stride, st);
  }
}

// (cos, sin) table of the online rotary for the rotation fused into the attention forward: row t holds cos of
// the D/2 angles pos[t] / theta^(2i/D) followed by their sines, from the same powf / sincosf as
// rotary_online_kernel (pos_encoding.cu:83-86), so a row rotated through the table is the row the rotary kernel
// would have written.
__global__ void __launch_bounds__(256) rotary_cos_sin_kernel(const int32_t* __restrict__ pos, float* __restrict__ cs,
                                                              int64_t tokens, int D, float theta) {
  const int half = D / 2;
  const int64_t n = tokens * half;
  for (int64_t it = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; it < n; it += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = it / half;
    const int i = (int)(it - t * half);
    const float ang = (float)pos[t] / powf(theta, (float)(2 * i) / (float)D);
    float sn, c;
    sincosf(ang, &sn, &c);
    cs[t * D + i] = c;
    cs[t * D + half + i] = sn;
  }
}

extern "C" int dgg_rotary_cos_sin(const int32_t* positions, float* cos_sin, int64_t tokens, int64_t head_dim,
                                  float rope_theta, void* stream) {
  DGG_REQUIRE(head_dim > 0 && head_dim % 16 == 0 && head_dim <= 512, DGG_ERR_UNSUPPORTED,
              "rotary_cos_sin: head_dim must be a positive multiple of 16 up to 512 (got %lld)", (long long)head_dim);
  DGG_REQUIRE(tokens >= 0 && tokens <= 0x7fffffff, DGG_ERR_SHAPE, "rotary_cos_sin: bad token count %lld",
              (long long)tokens);
  if (tokens == 0) return DGG_OK;
  DGG_REQUIRE(positions && cos_sin, DGG_ERR_NULL, "rotary_cos_sin: null pointer");
  const int64_t n = tokens * (head_dim / 2);
  const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(rotary_cos_sin_kernel, dim3(blocks), dim3(256), 0, dgg::as_stream(stream), positions, cos_sin,
                     tokens, (int)head_dim, rope_theta);
  return dgg::check_launch("rotary_cos_sin");
}

extern "C" int dgg_rotary_embedding_online(const int32_t* positions, void* query, void* key, int64_t tokens,
                                           int64_t head_num, int64_t kv_head_num, int64_t head_dim,
                                           int64_t q_row_stride, int64_t k_row_stride, int dtype, float rope_theta,
                                           void* stream) {
  DGG_REQUIRE(dgg::valid_dtype(dtype), DGG_ERR_DTYPE, "rotary_embedding_online: unsupported dtype code %d", dtype);
  DGG_REQUIRE(head_dim > 0 && head_dim % 16 == 0 && head_dim <= 512, DGG_ERR_UNSUPPORTED,
              "rotary_embedding_online: head_dim must be a positive multiple of 16 up to 512 (got %lld)",
              (long long)head_dim);
  DGG_REQUIRE(tokens >= 0 && tokens <= 0x7fffffff, DGG_ERR_SHAPE, "rotary_embedding_online: bad token count %lld",
              (long long)tokens);
  DGG_REQUIRE(head_num > 0 && kv_head_num >= 0 && head_num + kv_head_num <= 65536, DGG_ERR_SHAPE,
              "rotary_embedding_online: bad head counts %lld / %lld", (long long)head_num, (long long)kv_head_num);
  DGG_REQUIRE(q_row_stride >= head_num * head_dim, DGG_ERR_STRIDE,
              "rotary_embedding_online: query row stride %lld < head_num*head_dim", (long long)q_row_stride);
  if (key == nullptr) kv_head_num = 0;
  DGG_REQUIRE(kv_head_num == 0 || k_row_stride >= kv_head_num * head_dim, DGG_ERR_STRIDE,
              "rotary_embedding_online: key row stride %lld < kv_head_num*head_dim", (long long)k_row_stride);
  if (tokens == 0) return DGG_OK;
  DGG_REQUIRE(positions && query, DGG_ERR_NULL, "rotary_embedding_online: null pointer");
  hipStream_t st = dgg::as_stream(stream);
  switch (dtype) {
    case DGG_F16: return rotary_dispatch<F16>(positions, query, key, tokens, head_num, kv_head_num, head_dim, q_row_stride, k_row_stride, rope_theta, st);
    case DGG_BF16: return rotary_dispatch<BF16>(positions, query, key, tokens, head_num, kv_head_num, head_dim, q_row_stride, k_row_stride, rope_theta, st);
    default: return rotary_dispatch<F32>(positions, query, key, tokens, head_num, kv_head_num, head_dim, q_row_stride, k_row_stride, rope_theta, st);
  }
}
