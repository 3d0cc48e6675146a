// Top-k selection of the KV-cache policies: H2O's and SnapKV's top-k (torch.topk then a sort of the indices,
// models/h2o.py:51-52), either direction, and RoCo's whole selection (models/roco.py:54-61: the standard deviation
// of each key's attention probabilities, the n - recent smallest, the `recent` largest, the `budget` largest
// column sums among the smallest, concatenated and sorted) as one kernel.
//
// One 1024-thread workgroup per row; each thread keeps a contiguous segment of up to PER elements in registers.
// A selection is a radix select over an order-preserving 32-bit key (4 passes of 8 bits) that finds the k-th
// largest key K* among the candidate elements; every candidate with key > K* is taken, plus the lowest-indexed
// candidates equal to K* until k are taken. Block-wide exclusive scans over the contiguous segments give both the
// tie ranks and the output positions, so indices come out in ascending order without a sort.
//
// torch.topk leaves the order among equal values unspecified; these kernels define it: equal values are taken
// lowest index first, in either direction. NaN (either sign) ranks above +inf, as torch.topk and torch.sort rank
// it, and -0.0 equals +0.0.
#include "common.h"

namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;

struct TopkShared {
  uint32_t hist[kTopkWaves][256];
  uint32_t wsum[kTopkWaves];
  uint32_t sel_digit, sel_remaining;
};

// Key whose unsigned order is torch's order of fp32 values: NaN above +inf, -0.0 == +0.0.
__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) return 0xFFFFFFFFu;
  const uint32_t u = __float_as_uint(x == 0.f ? 0.f : x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide exclusive scan of one uint32 per thread (1024 threads = 16 waves); `total` gets the block sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wsum, uint32_t& total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t t = __shfl_up(inc, off, 64);
    if (lane >= off) inc += t;
  }
  if (lane == 63) wsum[wid] = inc;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int i = 0; i < kTopkWaves; ++i) {
    const uint32_t s = wsum[i];
    if (i < wid) before += s;
    all += s;
  }
  __syncthreads();
  total = all;
  return before + inc - v;
}

// Among this block's candidates (bit j of `cand`: element seg0 + j of the calling thread), marks the k with the
// largest keys, equal keys lowest index first, and returns the calling thread's take bits. k must not exceed the
// number of candidates. Histograms are per wave (no atomics shared across waves); the digit of each pass is found
// by a 256-thread suffix scan over the bins. Every thread of the block calls this with the same k.
template <int PER>
__device__ uint64_t radix_take(const uint32_t (&key)[PER], uint64_t cand, uint32_t k, TopkShared& sh) {
  if (k == 0) return 0;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t prefix = 0, pmask = 0, remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < kTopkWaves * 256; i += kTopkThreads) (&sh.hist[0][0])[i] = 0u;
    __syncthreads();
    if (shift == 24) {
      // The top byte (sign and leading exponent bits) of one row's scores is nearly constant, so most lanes of a
      // wave hit the same bin and their LDS atomics would serialise on one address: the lanes whose digit equals
      // the first active lane's add as one. The lower bytes spread over the bins, where this costs more than it
      // saves.
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const bool act = (cand >> j) & 1;
        const uint32_t d = key[j] >> 24;
        const uint64_t active = __ballot(act);
        if (active) {
          const int leader = __ffsll((long long)active) - 1;
          const uint32_t d0 = __shfl(d, leader, 64);
          const uint64_t same = __ballot(act && d == d0);
          if (lane == leader) atomicAdd(&sh.hist[wv][d0], (uint32_t)__popcll(same));
          else if (act && d != d0) atomicAdd(&sh.hist[wv][d], 1u);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (((cand >> j) & 1) && (key[j] & pmask) == prefix) atomicAdd(&sh.hist[wv][(key[j] >> shift) & 255u], 1u);
    }
    __syncthreads();
    // Thread t < 256 takes bin 255 - t: an inclusive scan over t counts the candidates in bins >= 255 - t.
    uint32_t c = 0, incl = 0;
    if (tid < 256) {
#pragma unroll
      for (int w2 = 0; w2 < kTopkWaves; ++w2) c += sh.hist[w2][255 - tid];
      incl = c;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
      }
      if (lane == 63) sh.wsum[wv] = incl;
    }
    __syncthreads();
    if (tid < 256) {
      uint32_t base = 0;
      for (int w2 = 0; w2 < wv; ++w2) base += sh.wsum[w2];
      const uint32_t hi = base + incl, lo = hi - c;  // candidates in bins above / from this bin
      if (lo < remaining && hi >= remaining) {      // exactly one bin: the k-th largest lies in it
        sh.sel_digit = 255u - (uint32_t)tid;
        sh.sel_remaining = remaining - lo;
      }
    }
    __syncthreads();
    prefix |= sh.sel_digit << shift;
    pmask |= 255u << shift;
    remaining = sh.sel_remaining;
  }
  // prefix = K*; `remaining` candidates equal to K* are still to be taken, lowest index first.
  uint32_t eq = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) eq += ((cand >> j) & 1) && key[j] == prefix;
  uint32_t tot;
  uint32_t eq_seen = block_exclusive_scan(eq, sh.wsum, tot);
  uint64_t take = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if ((cand >> j) & 1) {
      bool t = key[j] > prefix;
      if (key[j] == prefix) t = eq_seen++ < remaining;
      take |= (uint64_t)t << j;
    }
  }
  return take;
}

// Writes seg0 + j, (bit j of a) + (bit j of b) times, for every j of every thread, in ascending order to o[0, total).
__device__ __forceinline__ void write_taken(uint64_t a, uint64_t b, int seg0, int64_t* __restrict__ o, uint32_t total,
                                           TopkShared& sh) {
  uint32_t tot;
  uint32_t pos = block_exclusive_scan(__popcll(a) + __popcll(b), sh.wsum, tot);
  while (a | b) {
    const uint64_t low = (a | b) & (~(a | b) + 1);  // lowest element still to write
    const int j = __ffsll((long long)low) - 1;
    const int m = (int)((a >> j) & 1) + (int)((b >> j) & 1);
    for (int r = 0; r < m; ++r)
      if (pos < total) o[pos++] = seg0 + j;
    a &= ~low;
    b &= ~low;
  }
}

__device__ __forceinline__ void segment(int n, int& seg0, int& cnt, uint64_t& all) {
  const int per = (n + kTopkThreads - 1) / kTopkThreads;
  seg0 = min(n, (int)threadIdx.x * per);
  cnt = min(n, seg0 + per) - seg0;
  all = cnt >= 64 ? ~0ull : ((1ull << cnt) - 1);
}

// PER: elements per thread kept in registers (n <= PER * 1024).
template <int PER>
__global__ void __launch_bounds__(kTopkThreads) topk_kernel(const float* __restrict__ scores, int n, int k, int largest,
                                                             int64_t* __restrict__ out) {
  __shared__ TopkShared sh;
  const float* x = scores + (int64_t)blockIdx.x * n;
  int seg0, cnt;
  uint64_t all;
  segment(n, seg0, cnt, all);
  uint32_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    key[j] = j < cnt ? order_key(x[seg0 + j]) : 0u;
    if (!largest) key[j] = ~key[j];  // the smallest first; NaN (all ones) becomes the least
  }
  const uint64_t take = radix_take<PER>(key, all, (uint32_t)k, sh);
  write_taken(take, 0, seg0, out + (int64_t)blockIdx.x * k, (uint32_t)k, sh);
}

// roco_score / q_len, (roco_sq_score / q_len - (roco_score / q_len) ** 2) and its square root as torch computes them
// on the GPU: a tensor divided by a Python number is multiplied by the fp32 reciprocal, ** 2 is one multiply, sqrt is
// correctly rounded and a negative variance (cancellation) gives NaN. No fused multiply-add may merge these roundings.
__device__ __forceinline__ float roco_mean(float s1, float rcp) {
#pragma clang fp contract(off)
  return s1 * rcp;
}

__device__ __forceinline__ float roco_std(float s1, float s2, float rcp) {
#pragma clang fp contract(off)
  const float m = s1 * rcp;
  const float var = s2 * rcp - m * m;
  return __builtin_sqrtf(var);
}

// models/roco.py:54-61 for one row of roco_score / roco_sq_score: `recent` = the recent largest standard deviations,
// `other` = the n - recent smallest, `pick` = the budget largest roco_score / q_len among `other`; the output is the
// sorted concatenation of pick and recent (an index in both, possible only through ties, appears twice, as in the
// reference's cat + sort).
template <int PER>
__global__ void __launch_bounds__(kTopkThreads) roco_select_kernel(const float* __restrict__ s1,
                                                                    const float* __restrict__ s2, int n, float rcp,
                                                                    int recent, int budget, int64_t* __restrict__ out) {
  __shared__ TopkShared sh;
  const int64_t row = (int64_t)blockIdx.x * n;
  int seg0, cnt;
  uint64_t all;
  segment(n, seg0, cnt, all);
  uint32_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) key[j] = j < cnt ? order_key(roco_std(s1[row + seg0 + j], s2[row + seg0 + j], rcp)) : 0u;
  const uint64_t rec = radix_take<PER>(key, all, (uint32_t)recent, sh);       // roco.py:56
#pragma unroll
  for (int j = 0; j < PER; ++j) key[j] = ~key[j];
  const uint64_t other = radix_take<PER>(key, all, (uint32_t)(n - recent), sh);  // roco.py:55
#pragma unroll
  for (int j = 0; j < PER; ++j) key[j] = j < cnt ? order_key(roco_mean(s1[row + seg0 + j], rcp)) : 0u;
  const uint64_t pick = radix_take<PER>(key, other, (uint32_t)budget, sh);    // roco.py:57-58
  write_taken(pick, rec, seg0, out + (int64_t)blockIdx.x * (budget + recent), (uint32_t)(budget + recent), sh);
}

}  // namespace

extern "C" int dgg_topk_select(const float* scores, int64_t rows, int64_t n, int64_t k, int largest,
                               int64_t* out_idx, void* stream) {
  DGG_REQUIRE(rows >= 0 && rows < (1ll << 31), DGG_ERR_SHAPE, "topk_indices: bad row count %lld", (long long)rows);
  DGG_REQUIRE(n >= 1 && n <= 65536, DGG_ERR_SHAPE, "topk_indices: n must be in [1, 65536] (got %lld)", (long long)n);
  DGG_REQUIRE(k >= 1 && k <= n, DGG_ERR_SHAPE, "topk_indices: k must be in [1, n] (got k=%lld, n=%lld)",
              (long long)k, (long long)n);
  if (rows == 0) return DGG_OK;
  DGG_REQUIRE(scores && out_idx, DGG_ERR_NULL, "topk_indices: null pointer");
  const dim3 grid((unsigned)rows), block(kTopkThreads);
  hipStream_t st = dgg::as_stream(stream);
  const int lg = largest ? 1 : 0;
  if (n <= 4 * kTopkThreads)
    hipLaunchKernelGGL(topk_kernel<4>, grid, block, 0, st, scores, (int)n, (int)k, lg, out_idx);
  else if (n <= 16 * kTopkThreads)
    hipLaunchKernelGGL(topk_kernel<16>, grid, block, 0, st, scores, (int)n, (int)k, lg, out_idx);
  else
    hipLaunchKernelGGL(topk_kernel<64>, grid, block, 0, st, scores, (int)n, (int)k, lg, out_idx);
  return dgg::check_launch("topk_indices");
}

extern "C" int dgg_topk_indices(const float* scores, int64_t rows, int64_t n, int64_t k, int64_t* out_idx,
                                void* stream) {
  return dgg_topk_select(scores, rows, n, k, 1, out_idx, stream);
}

extern "C" int dgg_roco_select(const float* score, const float* sq_score, int64_t rows, int64_t n, int64_t q_len,
                               int64_t recent, int64_t budget, int64_t* out_idx, void* stream) {
  DGG_REQUIRE(rows >= 0 && rows < (1ll << 31), DGG_ERR_SHAPE, "roco_select: bad row count %lld", (long long)rows);
  DGG_REQUIRE(n >= 1 && n <= 65536, DGG_ERR_SHAPE, "roco_select: n must be in [1, 65536] (got %lld)", (long long)n);
  DGG_REQUIRE(q_len >= 1 && q_len <= (1ll << 24), DGG_ERR_SHAPE, "roco_select: q_len must be in [1, 2^24] (got %lld)",
              (long long)q_len);
  DGG_REQUIRE(recent >= 0 && recent <= n, DGG_ERR_SHAPE, "roco_select: recent must be in [0, n] (got %lld, n=%lld)",
              (long long)recent, (long long)n);
  DGG_REQUIRE(budget >= 0 && budget <= n - recent, DGG_ERR_SHAPE,
              "roco_select: budget must be in [0, n - recent] (got %lld, n=%lld, recent=%lld)", (long long)budget,
              (long long)n, (long long)recent);
  if (rows == 0 || budget + recent == 0) return DGG_OK;
  DGG_REQUIRE(score && sq_score && out_idx, DGG_ERR_NULL, "roco_select: null pointer");
  const float rcp = 1.0f / (float)q_len;  // torch's reciprocal of the Python divisor, in fp32
  const dim3 grid((unsigned)rows), block(kTopkThreads);
  hipStream_t st = dgg::as_stream(stream);
  const int r = (int)recent, b = (int)budget;
  if (n <= 4 * kTopkThreads)
    hipLaunchKernelGGL(roco_select_kernel<4>, grid, block, 0, st, score, sq_score, (int)n, rcp, r, b, out_idx);
  else if (n <= 16 * kTopkThreads)
    hipLaunchKernelGGL(roco_select_kernel<16>, grid, block, 0, st, score, sq_score, (int)n, rcp, r, b, out_idx);
  else
    hipLaunchKernelGGL(roco_select_kernel<64>, grid, block, 0, st, score, sq_score, (int)n, rcp, r, b, out_idx);
  return dgg::check_launch("roco_select");
}
