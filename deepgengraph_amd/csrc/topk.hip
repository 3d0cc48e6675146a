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
#include <algorithm>

#include "common.h"

namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;

struct TopkShared {
  uint32_t hist[256];
  uint32_t wsum[kTopkWaves];
  uint32_t sel_digit, sel_remaining, sel_whole;
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
// number of candidates. Every wave adds into one LDS histogram per pass, and a 256-thread suffix scan over its bins
// finds the pass's digit (per-wave histograms avoided the shared atomics but cost zeroing and reducing 16 x 256 bins
// per pass: measured on MI355X in an interleaved A/B, top-256 of 32 x 4,096 keys 9.85 -> 8.9 us, RoCo's selection at
// config-4 shapes 22.1 -> 20.1 us, top-256 of 32 x 1,048,576 154 -> 145.5 us). Every thread of the block calls this
// with the same k.
// The digit passes of radix_take: kstar = K*, the k-th largest candidate key (k >= 1), and `remaining` = the number
// of candidates equal to K* among the k. Unless `exact`, the passes stop as soon as the bin that holds the k-th key is
// taken whole: the k are then every candidate whose leading bytes are at least the digits chosen so far, and kstar is
// that prefix with zero lower bytes and `remaining` is 0xFFFFFFFF (every candidate equal to it is taken), which
// selects the same set (measured on MI355X in an interleaved A/B, two rounds: RoCo's selection at config-4 shapes
// 24.4 -> 22.0 us, top-256 of 32 x 1,048,576 keys 160 -> 154.5 us, of 32 x 4,096 10.2 -> 10.1 us).
template <int PER>
__device__ void radix_kstar(const uint32_t (&key)[PER], uint64_t cand, uint32_t k, TopkShared& sh, uint32_t& kstar,
                            uint32_t& remaining_out, bool exact = true) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t prefix = 0, pmask = 0, remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) sh.hist[tid] = 0u;
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
          if (lane == leader) atomicAdd(&sh.hist[d0], (uint32_t)__popcll(same));
          else if (act && d != d0) atomicAdd(&sh.hist[d], 1u);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (((cand >> j) & 1) && (key[j] & pmask) == prefix) atomicAdd(&sh.hist[(key[j] >> shift) & 255u], 1u);
    }
    __syncthreads();
    // Thread t < 256 takes bin 255 - t: an inclusive scan over t counts the candidates in bins >= 255 - t.
    uint32_t c = 0, incl = 0;
    if (tid < 256) {
      c = sh.hist[255 - tid];
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
        sh.sel_whole = hi == remaining;  // every candidate of the bin is among the k
      }
    }
    __syncthreads();
    prefix |= sh.sel_digit << shift;
    pmask |= 255u << shift;
    remaining = sh.sel_remaining;
    if (!exact && shift > 0 && sh.sel_whole) {  // (the same value in every thread: the whole block leaves together)
      remaining = 0xFFFFFFFFu;
      break;
    }
  }
  kstar = prefix;
  remaining_out = remaining;
}

template <int PER>
__device__ uint64_t radix_take(const uint32_t (&key)[PER], uint64_t cand, uint32_t k, TopkShared& sh,
                               uint32_t* bound = nullptr) {
  if (k == 0) return 0;
  uint32_t prefix, remaining;
  radix_kstar<PER>(key, cand, k, sh, prefix, remaining, bound != nullptr);
  if (bound != nullptr && threadIdx.x == 0) {  // K* and how many keys equal to it are taken
    bound[0] = prefix;
    bound[1] = remaining;
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

// As write_taken for one mask, writing idx[seg0 + j] in place of seg0 + j (positions ascending).
__device__ __forceinline__ void write_taken_gather(uint64_t a, int seg0, const int* __restrict__ idx,
                                                   int64_t* __restrict__ o, uint32_t total, TopkShared& sh) {
  uint32_t tot;
  uint32_t pos = block_exclusive_scan(__popcll(a), sh.wsum, tot);
  while (a) {
    const int j = __ffsll((long long)a) - 1;
    if (pos < total) o[pos++] = idx[seg0 + j];
    a &= a - 1;
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
  // roco.py:56 takes the `recent` largest std, roco.py:55 the n - recent smallest, both with equal keys lowest index
  // first. With K* the recent-th largest key, of which `recent` takes the first r, `other` is every key below K*
  // plus the first (c - r) of the c keys equal to it: one selection gives both masks. (A second selection of the
  // complemented keys measured 20.1 us against 16.5 us for this at config-4 shapes.)
  uint64_t rec = 0, other = all;
  if (recent > 0) {
    uint32_t kstar, r;
    radix_kstar<PER>(key, all, (uint32_t)recent, sh, kstar, r, true);
    uint32_t eq = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) eq += ((all >> j) & 1) && key[j] == kstar;
    uint32_t c;
    uint32_t seen = block_exclusive_scan(eq, sh.wsum, c);  // equal keys of the earlier threads (lower indices)
    other = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if ((all >> j) & 1) {
        const bool e = key[j] == kstar;
        rec |= (uint64_t)(key[j] > kstar || (e && seen < r)) << j;
        other |= (uint64_t)(key[j] < kstar || (e && seen < c - r)) << j;
        seen += e;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) key[j] = j < cnt ? order_key(roco_mean(s1[row + seg0 + j], rcp)) : 0u;
  const uint64_t pick = radix_take<PER>(key, other, (uint32_t)budget, sh);    // roco.py:57-58
  write_taken(pick, rec, seg0, out + (int64_t)blockIdx.x * (budget + recent), (uint32_t)(budget + recent), sh);
}

// ------------------------------------------------------------------------------------------------
// Rows longer than 65536 keys: the same selections (same key order, same tie rule, same output order) over many
// workgroups per row, through a caller-provided workspace, in one of two forms. A selection of k with
// ceil(n / kSel2Chunk) * k <= kSel2MaxCand runs in two stages (sel2_local_kernel, sel2_merge_kernel): each chunk's k
// largest as candidates, then k among those, reading the row once. Other selections run in passes: a row is cut into
// chunks of kSelChunk keys, one 256-thread workgroup per (chunk, row); wave w of a chunk owns its contiguous
// kSelWaveSpan keys, 64 at a time (lane l on key 64i + l), so a 64-bit ballot is one aligned word of a bit mask.
//   1. two histogram passes: pass p counts the candidates whose key matches the digits chosen so far into 256 bins
//      of its byte (LDS, then one global atomic per bin and workgroup); every workgroup of the next pass re-derives
//      the chosen digits from the finished histograms (a 256-bin suffix scan per pass);
//   2. the split at the 16-bit prefix P of K*, the k-th largest key: every candidate whose top 16 bits exceed P is
//      taken, its bit written straight into the selection's mask; the candidates whose top 16 bits equal P, the
//      only keys the remaining passes look at, go into a second bit mask (the prefix mask), and their third byte
//      into histogram pass 2;
//   3. histogram pass 3 over the prefix mask's keys;
//   4. per chunk, the number of prefix-mask keys equal to K*;
//   5. the rest of the selection: prefix-mask keys above K*, and those equal to K* while their rank among the equal
//      ones (counted over the earlier chunks, the earlier waves of the chunk and the earlier lanes) is below the
//      number still to take, i.e. lowest index first, OR'ed into the mask words of step 2; plus the mask's
//      population per chunk;
//   6. the indices of one or two masks in ascending order (an index in both written twice), each chunk at the sum of
//      the populations before it.
// Steps 1 and 2 read every key (three reads of the row); steps 3-5 load only the keys of mask words that hold a
// prefix-mask bit, which for scores in general is a small share of the row (all of it when every key is equal).
// RoCo chains three selections: `recent` (largest std), `other` (smallest std), `pick` (largest mean among the
// candidates of `other`'s mask), then writes pick and recent merged. When `recent` and `pick` both fit the two-stage
// form, they take it (their sorted lists go to the output rows and roco_merge_kernel merges them), and `other`, whose
// k is n - recent, is built from `recent`'s boundary by steps 4 and 5 alone (sel_complement_run); otherwise all three
// run in passes.
// ------------------------------------------------------------------------------------------------
constexpr int kSelThreads = 256;
constexpr int kSelPer = 16;                                 // keys per lane per chunk, loaded back to back
constexpr int kSelWaveSpan = 64 * kSelPer;                  // keys per wave per chunk
constexpr int kSelChunk = kSelWaveSpan * (kSelThreads / 64);  // keys per workgroup
constexpr int kSelMaxN = 1 << 26;
constexpr int kSelNSel = 3;                                 // selections a workspace holds (RoCo's three)
// Two-stage top-k (small k): each 1024-thread workgroup takes the k largest of its kSel2Chunk keys, then one workgroup
// per row selects among the chunks' candidates (at most kSel2MaxCand, held in registers by topk's kernels). 8 keys per
// lane fit 64 VGPRs, so two workgroups share a CU (measured on MI355X, top-256 of 32 rows: 186-187 against 205 us at
// 1,048,576 keys, 31.8 against 33.4 us at 131,072, for 16 keys per lane at 128 VGPRs and one workgroup per CU, both
// with the 64-per-lane merge; 32 keys per lane spill 124 VGPRs and 164 SGPRs).
constexpr int kSel2Per = 8;                                 // keys per lane in the first stage
constexpr int kSel2Chunk = 64 * kSel2Per * kTopkWaves;      // keys per workgroup
constexpr int kSel2MaxCand = 64 * kTopkThreads;             // candidates per row
constexpr int kSel2C2 = 16384;  // second-level candidates per row (groups * k <= 65,536 / 8 + k, see sel2_run)

struct SelWs {
  uint32_t* hist;   // [rows][kSelNSel][4][256]
  uint32_t* eqcnt;  // [rows][kSelNSel][chunks]
  uint32_t* mcnt;   // [rows][kSelNSel][chunks]
  uint64_t* mask;   // [rows][kSelNSel][words]
  uint64_t* pre;    // [rows][words]: the prefix mask of the selection in progress
  uint32_t* ckey;   // two-stage candidates, [rows][m] with m = chunks * k <= kSel2MaxCand (room for kSel2MaxCand per row)
  int* cidx;        // their indices, same layout
  uint32_t* c2key;  // the group level's candidates, [rows][kSel2C2]
  int* c2idx;       // their indices
  int chunks, words;
  int spc;          // kSelChunk-key sub-chunks per workgroup (a chunk is spc * kSelChunk keys)
};

__host__ __device__ inline int64_t sel_align(int64_t x) { return (x + 255) & ~(int64_t)255; }

// Workspace layout for `rows` rows of n keys; returns the total byte count (ws may be null to size only). A workgroup
// takes enough sub-chunks that there are about 2048 workgroups in all: more would multiply the global histogram
// atomics on the same 256 bins per row, fewer would leave the chip idle.
inline int64_t sel_layout(int64_t rows, int64_t n, void* base, SelWs* ws) {
  const int64_t sub = (n + kSelChunk - 1) / kSelChunk;
  const int64_t want = std::max<int64_t>(1, (2048 + rows - 1) / std::max<int64_t>(rows, 1));
  const int64_t spc = std::max<int64_t>(1, (sub + want - 1) / want);
  const int64_t chunks = (sub + spc - 1) / spc, words = (n + 63) / 64;
  const int64_t hist_b = sel_align(rows * kSelNSel * 1024 * 4);
  const int64_t cnt_b = sel_align(rows * kSelNSel * chunks * 4);
  const int64_t mask_b = sel_align(rows * kSelNSel * words * 8);
  const int64_t pre_b = sel_align(rows * words * 8);
  const int64_t cand_b = sel_align(rows * (int64_t)kSel2MaxCand * 4);
  const int64_t cand2_b = sel_align(rows * (int64_t)kSel2C2 * 4);
  if (ws != nullptr) {
    char* c = static_cast<char*>(base);
    ws->hist = reinterpret_cast<uint32_t*>(c);
    ws->eqcnt = reinterpret_cast<uint32_t*>(c + hist_b);
    ws->mcnt = reinterpret_cast<uint32_t*>(c + hist_b + cnt_b);
    ws->mask = reinterpret_cast<uint64_t*>(c + hist_b + 2 * cnt_b);
    ws->pre = reinterpret_cast<uint64_t*>(c + hist_b + 2 * cnt_b + mask_b);
    ws->ckey = reinterpret_cast<uint32_t*>(c + hist_b + 2 * cnt_b + mask_b + pre_b);
    ws->cidx = reinterpret_cast<int*>(c + hist_b + 2 * cnt_b + mask_b + pre_b + cand_b);
    ws->c2key = reinterpret_cast<uint32_t*>(c + hist_b + 2 * cnt_b + mask_b + pre_b + 2 * cand_b);
    ws->c2idx = reinterpret_cast<int*>(c + hist_b + 2 * cnt_b + mask_b + pre_b + 2 * cand_b + cand2_b);
    ws->chunks = (int)chunks;
    ws->words = (int)words;
    ws->spc = (int)spc;
  }
  return hist_b + 2 * cnt_b + mask_b + pre_b + 2 * cand_b + 2 * cand2_b;
}

// Key sources: element j of row `row` as an order key (larger = taken first), in two steps: load() reads what the
// key is made from, key() forms it (so that a caller can issue every load before it waits for any).
struct KeyScores {  // topk_kernel's key: the score, complemented for the smallest-first direction
  typedef float raw_t;
  const float* x;
  int n, largest;
  __device__ __forceinline__ raw_t load(int64_t row, int j) const { return x[row * n + j]; }
  __device__ __forceinline__ uint32_t key(raw_t v) const {
    const uint32_t k = order_key(v);
    return largest ? k : ~k;
  }
};
struct KeyStd {  // roco_select_kernel's std key (complemented: the smallest first)
  typedef f32x2 raw_t;
  const float* s1;
  const float* s2;
  int n;
  float rcp;
  int complement;
  __device__ __forceinline__ raw_t load(int64_t row, int j) const { return f32x2{s1[row * n + j], s2[row * n + j]}; }
  __device__ __forceinline__ uint32_t key(raw_t v) const {
    const uint32_t k = order_key(roco_std(v[0], v[1], rcp));
    return complement ? ~k : k;
  }
};
struct KeyMean {  // roco_select_kernel's third key: roco_score / q_len
  typedef float raw_t;
  const float* s1;
  int n;
  float rcp;
  __device__ __forceinline__ raw_t load(int64_t row, int j) const { return s1[row * n + j]; }
  __device__ __forceinline__ uint32_t key(raw_t v) const { return order_key(roco_mean(v, rcp)); }
};

struct SelShared {
  uint32_t hist[256];
  uint32_t wsum[kSelThreads / 64];
  uint32_t digit, rem;
};

// Digits chosen by the finished histogram passes 0 .. np-1 of a selection of k: prefix / pmask of the key bits
// fixed so far and the number of candidates still to take among those matching them. All 256 threads call it.
__device__ void sel_state(const uint32_t* H, int np, uint32_t k, uint32_t& prefix, uint32_t& pmask, uint32_t& rem,
                          SelShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  prefix = 0;
  pmask = 0;
  rem = k;
  for (int ps = 0; ps < np; ++ps) {
    const uint32_t c = H[ps * 256 + 255 - tid];  // thread t takes bin 255 - t
    uint32_t incl = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    if (lane == 63) sh.wsum[wv] = incl;
    __syncthreads();
    uint32_t base = 0;
    for (int w2 = 0; w2 < wv; ++w2) base += sh.wsum[w2];
    const uint32_t hi = base + incl, lo = hi - c;
    if (lo < rem && hi >= rem) {
      sh.digit = 255u - (uint32_t)tid;
      sh.rem = rem - lo;
    }
    __syncthreads();
    const int shift = 24 - 8 * ps;
    prefix |= sh.digit << shift;
    pmask |= 255u << shift;
    rem = sh.rem;
    __syncthreads();
  }
}

// Candidate sets of a pass: every key (kSelAll), the prefix mask (kSelPrefix), or the mask of an earlier selection.
constexpr int kSelAll = -1, kSelPrefix = -2;
__device__ __forceinline__ const uint64_t* sel_cmask(const SelWs& ws, int64_t row, int cand) {
  if (cand == kSelPrefix) return ws.pre + row * ws.words;
  return cand < 0 ? nullptr : ws.mask + (row * kSelNSel + cand) * ws.words;
}
// A two-stage selection's boundary of row `row`, {K*, keys equal to K* taken}, kept in the first two words of the row's
// selection-0 histogram (which a two-stage selection does not use).
__device__ __forceinline__ uint32_t* sel_bound(const SelWs& ws, int64_t row) { return ws.hist + row * kSelNSel * 1024; }

__global__ void __launch_bounds__(256) sel_zero_kernel(uint32_t* p, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) p[i] = 0u;
}

// The keys of this lane in its wave's span (key j0 + 64 i for i < kSelPer, j0 - lane a multiple of 64), all loads
// issued before any is used; bit i of the result: the key exists and is a candidate. With a candidate mask, step i
// covers exactly mask word (j0 - lane) / 64 + i: its words are loaded first (one per lane), a step whose word is zero
// issues no load, and only the lanes of candidates load their key.
template <class KeyF>
__device__ __forceinline__ uint32_t sel_load(const KeyF& kf, int64_t row, int j0, int n, const uint64_t* cm,
                                             uint32_t (&key)[kSelPer]) {
  uint32_t valid = 0;
  if (cm == nullptr) {
#pragma unroll
    for (int i = 0; i < kSelPer; ++i) {
      const int j = j0 + 64 * i;
      const bool ok = j < n;
      key[i] = ok ? kf.key(kf.load(row, j)) : 0u;
      valid |= (uint32_t)ok << i;
    }
    return valid;
  }
  const int lane = threadIdx.x & 63;
  const int w0 = (j0 - lane) >> 6, nwords = (n + 63) >> 6;
  const uint64_t mine = lane < kSelPer && w0 + lane < nwords ? cm[w0 + lane] : 0ull;
  static_assert(kSelPer <= 64, "one candidate word per lane");
  typename KeyF::raw_t raw[kSelPer];
#pragma unroll
  for (int i = 0; i < kSelPer; ++i) {
    // (readlane returns a signed int: each half goes through uint32_t so that the low half is not sign-extended)
    const uint64_t cw = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(mine >> 32), i) << 32) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)mine, i);
    const bool c = (cw >> lane) & 1ull;  // a mask bit is never set past n
    raw[i] = typename KeyF::raw_t{};
    if (cw != 0ull && c) raw[i] = kf.load(row, j0 + 64 * i);  // only the candidates' lanes load
    valid |= (uint32_t)c << i;
  }
#pragma unroll
  for (int i = 0; i < kSelPer; ++i) key[i] = (valid >> i) & 1 ? kf.key(raw[i]) : 0u;
  return valid;
}

// Adds digit d of every lane with m set to the LDS histogram: the lanes sharing the first active lane's digit add as
// one atomic, then those sharing the next remaining lane's digit, and the rest one atomic each (a wave's leading bytes
// mostly fall in one or two bins, where per-lane atomics on one LDS address serialise).
__device__ __forceinline__ void sel_hist_add(uint32_t* hist, bool m, uint32_t d) {
  const int lane = threadIdx.x & 63;
  uint64_t active = __ballot(m);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    if (active == 0ull) return;
    const int leader = __ffsll((long long)active) - 1;
    const uint32_t d0 = __shfl(d, leader, 64);
    const uint64_t same = __ballot(((active >> lane) & 1ull) && d == d0);
    if (lane == leader) atomicAdd(&hist[d0], (uint32_t)__popcll(same));
    active &= ~same;
  }
  if ((active >> lane) & 1ull) atomicAdd(&hist[d], 1u);
}

// Pass `ps` of the histogram of selection `sel` (k of the candidates: every key, or the bits of selection cand_sel).
template <class KeyF>
__global__ void __launch_bounds__(kSelThreads) sel_hist_kernel(KeyF kf, int n, SelWs ws, int sel, int ps, uint32_t k,
                                                                int cand_sel) {
  __shared__ SelShared sh;
  const int64_t row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t* H = ws.hist + (row * kSelNSel + sel) * 1024;
  const uint64_t* cm = sel_cmask(ws, row, cand_sel);
  uint32_t prefix, pmask, rem;
  sel_state(H, ps, k, prefix, pmask, rem, sh);
  sh.hist[tid] = 0u;
  __syncthreads();
  const int shift = 24 - 8 * ps;
  for (int sc = 0; sc < ws.spc; ++sc) {
    uint32_t key[kSelPer];
    const uint32_t valid =
        sel_load(kf, row, (blockIdx.x * ws.spc + sc) * kSelChunk + wv * kSelWaveSpan + lane, n, cm, key);
#pragma unroll
    for (int i = 0; i < kSelPer; ++i) {
      const bool m = ((valid >> i) & 1) && (key[i] & pmask) == prefix;
      const uint32_t d = (key[i] >> shift) & 255u;
      sel_hist_add(sh.hist, m, d);
    }
  }
  __syncthreads();
  if (sh.hist[tid] != 0u) atomicAdd(&H[ps * 256 + tid], sh.hist[tid]);
}

// Step 2 of a selection of k (k >= 1): with the digits of histogram passes 0 and 1 chosen, the 16-bit prefix P of K*.
// Candidates whose top 16 bits exceed P are taken (their bits are the selection's mask words as written here);
// candidates whose top 16 bits equal P form the prefix mask, and their bits 15..8 go into histogram pass 2. Every
// mask word of the chunk is written, in both masks.
template <class KeyF>
__global__ void __launch_bounds__(kSelThreads) sel_split_kernel(KeyF kf, int n, SelWs ws, int sel, uint32_t k,
                                                                 int cand_sel) {
  __shared__ SelShared sh;
  const int64_t row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t* H = ws.hist + (row * kSelNSel + sel) * 1024;
  const uint64_t* cm = sel_cmask(ws, row, cand_sel);
  uint64_t* out = ws.mask + (row * kSelNSel + sel) * ws.words;
  uint64_t* pre = ws.pre + row * ws.words;
  uint32_t prefix, pmask, rem;
  sel_state(H, 2, k, prefix, pmask, rem, sh);
  sh.hist[tid] = 0u;
  __syncthreads();
  const uint32_t p16 = prefix >> 16;
  for (int sc = 0; sc < ws.spc; ++sc) {
    const int js = (blockIdx.x * ws.spc + sc) * kSelChunk + wv * kSelWaveSpan;  // first key of this wave
    uint32_t key[kSelPer];
    const uint32_t valid = sel_load(kf, row, js + lane, n, cm, key);
#pragma unroll
    for (int i = 0; i < kSelPer; ++i) {
      const bool v = (valid >> i) & 1;
      const uint32_t top = key[i] >> 16;
      const uint64_t am = __ballot(v && top > p16);
      const bool m = v && top == p16;
      const uint64_t pm = __ballot(m);
      const int jw = js + 64 * i;
      if (lane == 0 && jw < n) {
        out[jw >> 6] = am;
        pre[jw >> 6] = pm;
      }
      sel_hist_add(sh.hist, m, (key[i] >> 8) & 255u);  // histogram pass 2
    }
  }
  __syncthreads();
  if (sh.hist[tid] != 0u) atomicAdd(&H[2 * 256 + tid], sh.hist[tid]);
}

// Candidates equal to K* per chunk. comp: K* is the complement of the K* of the two-stage selection whose boundary
// sel_bound holds (see sel_mark_kernel).
template <class KeyF>
__global__ void __launch_bounds__(kSelThreads) sel_eqcount_kernel(KeyF kf, int n, SelWs ws, int sel, uint32_t k,
                                                                   int cand_sel, int comp) {
  __shared__ SelShared sh;
  const int64_t row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t* cm = sel_cmask(ws, row, cand_sel);
  uint32_t kstar, pmask, rem;
  if (comp) kstar = ~sel_bound(ws, row)[0];
  else sel_state(ws.hist + (row * kSelNSel + sel) * 1024, 4, k, kstar, pmask, rem, sh);
  uint32_t eq = 0;
  for (int sc = 0; sc < ws.spc; ++sc) {
    uint32_t key[kSelPer];
    const uint32_t valid =
        sel_load(kf, row, (blockIdx.x * ws.spc + sc) * kSelChunk + wv * kSelWaveSpan + lane, n, cm, key);
#pragma unroll
    for (int i = 0; i < kSelPer; ++i) eq += ((valid >> i) & 1) && key[i] == kstar;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) eq += __shfl_xor(eq, off, 64);
  if (lane == 0) sh.wsum[wv] = eq;
  __syncthreads();
  if (tid == 0) ws.eqcnt[(row * kSelNSel + sel) * ws.chunks + blockIdx.x] = sh.wsum[0] + sh.wsum[1] + sh.wsum[2] + sh.wsum[3];
}

// Sum of cnt[0 .. m) over the workgroup (every thread gets it).
__device__ __forceinline__ uint32_t sel_block_sum(const uint32_t* cnt, int m, SelShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t v = 0;
  for (int c = tid; c < m; c += kSelThreads) v += cnt[c];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if (lane == 0) sh.wsum[wv] = v;
  __syncthreads();
  const uint32_t s = sh.wsum[0] + sh.wsum[1] + sh.wsum[2] + sh.wsum[3];
  __syncthreads();
  return s;
}

// The selection's bit mask and its population per chunk. k == 0 selects nothing. merge: OR the bits taken here into
// the mask words already written by sel_split_kernel (the keys above the prefix). comp: the selection of the n - r
// smallest keys (in KeyF's complemented order, the n - r largest) when a two-stage selection took the r largest and
// left its boundary {K*, e taken equal to K*} in sel_bound: its K* is ~K* and it takes the first (equal count - e)
// keys equal to it (with no histogram passes; sel_eqcount_kernel with comp counts the equal keys first). Both take
// equal keys lowest index first, so the two sets are complements except where the equal keys overlap.
template <class KeyF>
__global__ void __launch_bounds__(kSelThreads) sel_mark_kernel(KeyF kf, int n, SelWs ws, int sel, uint32_t k,
                                                                int cand_sel, int merge, int comp) {
  __shared__ SelShared sh;
  __shared__ uint32_t weq[kSelThreads / 64];
  const int64_t row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t* cm = sel_cmask(ws, row, cand_sel);
  uint64_t* out = ws.mask + (row * kSelNSel + sel) * ws.words;
  uint32_t kstar = 0, pmask, rem = 0, eq_before = 0;
  if (k > 0) {
    const uint32_t* eqc = ws.eqcnt + (row * kSelNSel + sel) * ws.chunks;
    if (comp) {
      const uint32_t* bnd = sel_bound(ws, row);
      kstar = ~bnd[0];
      rem = sel_block_sum(eqc, ws.chunks, sh) - bnd[1];
    } else {
      sel_state(ws.hist + (row * kSelNSel + sel) * 1024, 4, k, kstar, pmask, rem, sh);
    }
    eq_before = sel_block_sum(eqc, blockIdx.x, sh);
  }
  // sub-chunk by sub-chunk, in key order: this lane's keys above / equal to K* (one bit per step), the equal ones'
  // ranks counted over the earlier sub-chunks, waves and lanes
  const uint64_t lt = (1ull << lane) - 1;
  uint32_t rank_base = eq_before, taken = 0;
  for (int sc = 0; sc < ws.spc; ++sc) {
    const int js = (blockIdx.x * ws.spc + sc) * kSelChunk + wv * kSelWaveSpan;  // first key of this wave
    // merge: the wave's kSelPer mask words as sel_split_kernel wrote them, one per lane, read before any is rewritten
    const uint64_t above = merge && lane < kSelPer && (js >> 6) + lane < ws.words ? out[(js >> 6) + lane] : 0ull;
    uint32_t gtb = 0, eqb = 0, weq_cnt = 0;
    if (k > 0) {
      uint32_t key[kSelPer];
      const uint32_t valid = sel_load(kf, row, js + lane, n, cm, key);
#pragma unroll
      for (int i = 0; i < kSelPer; ++i) {
        const bool v = (valid >> i) & 1;
        gtb |= (uint32_t)(v && key[i] > kstar) << i;
        eqb |= (uint32_t)(v && key[i] == kstar) << i;
      }
      weq_cnt = __popc(eqb);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) weq_cnt += __shfl_xor(weq_cnt, off, 64);
    }
    if (lane == 0) weq[wv] = weq_cnt;
    __syncthreads();
    uint32_t rank = rank_base;
    for (int w2 = 0; w2 < wv; ++w2) rank += weq[w2];
    rank_base += weq[0] + weq[1] + weq[2] + weq[3];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSelPer; ++i) {
      const int jw = js + 64 * i;  // first key of this step
      if (jw < n) {
        const bool e = (eqb >> i) & 1;
        const uint64_t em = __ballot(e);
        const uint32_t my_rank = rank + (uint32_t)__popcll(em & lt);
        const bool take = ((gtb >> i) & 1) || (e && my_rank < rem);
        const uint64_t ab = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(above >> 32), i) << 32) |
                            (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)above, i);
        const uint64_t tm = __ballot(take) | ab;
        rank += (uint32_t)__popcll(em);
        taken += (uint32_t)__popcll(tm);
        if (lane == 0) out[jw >> 6] = tm;
      }
    }
  }
  __syncthreads();
  if (lane == 0) sh.wsum[wv] = taken;
  __syncthreads();
  if (tid == 0) ws.mcnt[(row * kSelNSel + sel) * ws.chunks + blockIdx.x] = sh.wsum[0] + sh.wsum[1] + sh.wsum[2] + sh.wsum[3];
}

// Indices of mask A (and B, -1 = none) in ascending order into out [rows, out_k]; an index in both appears twice.
__global__ void __launch_bounds__(kSelThreads) sel_emit_kernel(int n, SelWs ws, int sel_a, int sel_b,
                                                                int64_t* __restrict__ out, int out_k) {
  __shared__ SelShared sh;
  __shared__ uint32_t wtot[kSelThreads / 64];
  const int64_t row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t* ma = ws.mask + (row * kSelNSel + sel_a) * ws.words;
  const uint64_t* mb = sel_b < 0 ? nullptr : ws.mask + (row * kSelNSel + sel_b) * ws.words;
  uint32_t base = sel_block_sum(ws.mcnt + (row * kSelNSel + sel_a) * ws.chunks, blockIdx.x, sh);
  if (sel_b >= 0) base += sel_block_sum(ws.mcnt + (row * kSelNSel + sel_b) * ws.chunks, blockIdx.x, sh);
  static_assert(kSelWaveSpan / 64 <= 64, "one mask word per lane");
  const uint64_t lt = (1ull << lane) - 1;
  int64_t* o = out + row * out_k;
  for (int sc = 0; sc < ws.spc; ++sc) {
    const int w0 = ((blockIdx.x * ws.spc + sc) * kSelChunk + wv * kSelWaveSpan) >> 6;  // first mask word of the wave
    const int nwd = max(0, min(ws.words, w0 + kSelWaveSpan / 64) - w0);               // its words (one per lane)
    const uint64_t my_a = lane < nwd ? ma[w0 + lane] : 0ull, my_b = mb && lane < nwd ? mb[w0 + lane] : 0ull;
    uint32_t tot = __popcll(my_a) + __popcll(my_b);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) tot += __shfl_xor(tot, off, 64);
    if (lane == 0) wtot[wv] = tot;
    __syncthreads();
    uint32_t pos0 = base;
    for (int w2 = 0; w2 < wv; ++w2) pos0 += wtot[w2];
    base += wtot[0] + wtot[1] + wtot[2] + wtot[3];
    __syncthreads();
    for (int i = 0; i < nwd; ++i) {
      const int w = w0 + i;
      const uint64_t a = __shfl(my_a, i, 64), b = __shfl(my_b, i, 64);
      if ((a | b) == 0) continue;
      const int ba = (int)((a >> lane) & 1), bb = (int)((b >> lane) & 1);
      uint32_t pos = pos0 + (uint32_t)(__popcll(a & lt) + __popcll(b & lt));
      const int64_t j = (int64_t)w * 64 + lane;
      for (int r = 0; r < ba + bb; ++r, ++pos)
        if (pos < (uint32_t)out_k) o[pos] = j;
      pos0 += (uint32_t)(__popcll(a) + __popcll(b));
    }
  }
}

// Two-stage top-k, stage 1: the k largest candidate keys of chunk blockIdx.x (kSel2Chunk keys; wave w owns the
// contiguous kSel2Span keys from w * kSel2Span, lane l the keys l + 64 i; the candidates are every key, or the bits
// of an earlier selection's mask), equal keys lowest index first, written as (key, index) in ascending index order to
// the chunk's k candidate slots. A chunk of fewer than k candidates fills its remaining slots with key 0, which is
// never taken: the row holds at least k candidates, and every key is above 0 (order keys of the largest-first
// direction; NaN maps to the top) or, for KeyScores' smallest-first keys, where NaN maps to 0, without a mask only
// the last chunk pads, after every other slot, and among equal keys the lowest slot goes first.
template <class KeyF>
__global__ void __launch_bounds__(kTopkThreads) __attribute__((amdgpu_waves_per_eu(8)))
sel2_local_kernel(KeyF kf, int n, int k, SelWs ws, int cand_sel) {
  constexpr int kSel2Span = 64 * kSel2Per;  // keys per wave
  __shared__ TopkShared sh;
  __shared__ uint32_t wcnt[kTopkWaves];
  const int64_t row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c0 = blockIdx.x * kSel2Chunk;
  const int j0 = c0 + wv * kSel2Span + lane;
  uint32_t key[kSel2Per];
  uint64_t valid = 0;
  const uint64_t* cm = sel_cmask(ws, row, cand_sel);
  if constexpr (sizeof(typename KeyF::raw_t) == 4) {
    // the loaded bits first, then the keys (in place, so that both fit the register budget)
#pragma unroll
    for (int i = 0; i < kSel2Per; ++i)
      key[i] = j0 + 64 * i < n ? __builtin_bit_cast(uint32_t, kf.load(row, j0 + 64 * i)) : 0u;
#pragma unroll
    for (int i = 0; i < kSel2Per; ++i) {
      const bool ok = j0 + 64 * i < n;
      key[i] = ok ? kf.key(__builtin_bit_cast(typename KeyF::raw_t, key[i])) : 0u;
      valid |= (uint64_t)ok << i;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSel2Per; ++i) {
      const bool ok = j0 + 64 * i < n;
      key[i] = ok ? kf.key(kf.load(row, j0 + 64 * i)) : 0u;
      valid |= (uint64_t)ok << i;
    }
  }
  uint32_t cnt_chunk = (uint32_t)min(kSel2Chunk, n - c0);
  if (cm != nullptr) {  // candidates: the mask's bits (step i covers mask word (j0 - lane) / 64 + i)
    const int w0 = (j0 - lane) >> 6, nwords = (n + 63) >> 6;
    const uint64_t mine = lane < kSel2Per && w0 + lane < nwords ? cm[w0 + lane] : 0ull;
    uint32_t vmask = 0;
#pragma unroll
    for (int i = 0; i < kSel2Per; ++i) {
      const uint64_t cw = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(mine >> 32), i) << 32) |
                          (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)mine, i);
      vmask |= (uint32_t)((cw >> lane) & 1ull) << i;
    }
    valid &= vmask;
    uint32_t c = __popc((uint32_t)valid);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off, 64);
    if (lane == 0) wcnt[wv] = c;
    __syncthreads();
    cnt_chunk = 0;
    for (int w2 = 0; w2 < kTopkWaves; ++w2) cnt_chunk += wcnt[w2];
    __syncthreads();
  }
  const uint32_t kk = min((uint32_t)k, cnt_chunk);  // k <= the chunk's candidates, or all of them
  const int64_t slot0 = (row * gridDim.x + blockIdx.x) * (int64_t)k;
  uint32_t* ck = ws.ckey + slot0;
  int* ci = ws.cidx + slot0;
  for (int q = (int)kk + tid; q < k; q += kTopkThreads) {
    ck[q] = 0u;
    ci[q] = 0;
  }
  if (kk == 0) return;  // (uniform over the workgroup)
  uint32_t kstar, rem;
  radix_kstar<kSel2Per>(key, valid, kk, sh, kstar, rem, false);
  // ranks of the keys equal to K* in index order (wave, step, lane), then the taken keys' slots in the same order
  const uint64_t lt = (1ull << lane) - 1;
  uint32_t eqb = 0, weq = 0;
#pragma unroll
  for (int i = 0; i < kSel2Per; ++i) {
    const bool e = ((valid >> i) & 1) && key[i] == kstar;
    eqb |= (uint32_t)e << i;
    weq += (uint32_t)__popcll(__ballot(e));
  }
  if (lane == 0) wcnt[wv] = weq;
  __syncthreads();
  uint32_t rank = 0;
  for (int w2 = 0; w2 < wv; ++w2) rank += wcnt[w2];
  __syncthreads();
  uint32_t takeb = 0, wtake = 0;
#pragma unroll
  for (int i = 0; i < kSel2Per; ++i) {
    const bool e = (eqb >> i) & 1;
    const uint64_t em = __ballot(e);
    const bool t = (((valid >> i) & 1) && key[i] > kstar) || (e && rank + (uint32_t)__popcll(em & lt) < rem);
    rank += (uint32_t)__popcll(em);
    takeb |= (uint32_t)t << i;
    wtake += (uint32_t)__popcll(__ballot(t));
  }
  if (lane == 0) wcnt[wv] = wtake;
  __syncthreads();
  uint32_t pos = 0;
  for (int w2 = 0; w2 < wv; ++w2) pos += wcnt[w2];
#pragma unroll
  for (int i = 0; i < kSel2Per; ++i) {
    const bool t = (takeb >> i) & 1;
    const uint64_t tm = __ballot(t);
    if (t) {
      const uint32_t p = pos + (uint32_t)__popcll(tm & lt);
      ck[p] = key[i];
      ci[p] = j0 + 64 * i;
    }
    pos += (uint32_t)__popcll(tm);
  }
}

// Two-stage top-k, stage 2: the k largest of a row's m candidates (row stride crs; slot order = index order, lowest
// slot first on equal keys), their indices written in ascending order; with `bound` set, also the row's K* and the
// number of keys equal to it that were taken (sel_bound).
template <int PER>
__global__ void __launch_bounds__(kTopkThreads) sel2_merge_kernel(SelWs ws, const uint32_t* __restrict__ ckey,
                                                                   const int* __restrict__ cidx, int64_t crs, int m,
                                                                   int k, int64_t* __restrict__ out, int64_t out_rs,
                                                                   int bound) {
  __shared__ TopkShared sh;
  const uint32_t* kp = ckey + (int64_t)blockIdx.x * crs;
  const int* ip = cidx + (int64_t)blockIdx.x * crs;
  int seg0, cnt;
  uint64_t all;
  segment(m, seg0, cnt, all);
  uint32_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) key[j] = j < cnt ? kp[seg0 + j] : 0u;
  const uint64_t take =
      radix_take<PER>(key, all, (uint32_t)k, sh, bound ? sel_bound(ws, blockIdx.x) : nullptr);
  write_taken_gather(take, seg0, ip, out + (int64_t)blockIdx.x * out_rs, (uint32_t)k, sh);
}

// The group level between the two stages, for rows with many chunks: workgroup (g, row) takes the k largest of the
// candidates in slots [g * gslots, (g + 1) * gslots) of the row (whole chunks, so at least k of them) and writes them
// as (key, index) in slot order to slots [g * k, (g + 1) * k) of the row's group-level candidates. The groups of a
// row run side by side instead of one workgroup per row walking all of them.
template <int PER>
__global__ void __launch_bounds__(kTopkThreads) sel2_group_kernel(SelWs ws, int m, int k, int gslots) {
  __shared__ TopkShared sh;
  const int64_t row = blockIdx.y;
  const int s0 = blockIdx.x * gslots;
  const int cnt_g = min(gslots, m - s0);
  const uint32_t* kp = ws.ckey + row * m + s0;
  const int* ip = ws.cidx + row * m + s0;
  int seg0, cnt;
  uint64_t all;
  segment(cnt_g, seg0, cnt, all);
  uint32_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) key[j] = j < cnt ? kp[seg0 + j] : 0u;
  uint64_t take = radix_take<PER>(key, all, (uint32_t)k, sh);
  uint32_t tot;
  uint32_t pos = block_exclusive_scan(__popcll(take), sh.wsum, tot);
  uint32_t* ok = ws.c2key + row * kSel2C2 + (int64_t)blockIdx.x * k;
  int* oi = ws.c2idx + row * kSel2C2 + (int64_t)blockIdx.x * k;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if ((take >> j) & 1) {
      ok[pos] = key[j];
      oi[pos] = ip[seg0 + j];
      ++pos;
    }
  }
}

template <int PER>
void sel2_merge_launch(const SelWs& ws, const uint32_t* ck, const int* ci, int64_t crs, int rows, int m, int k,
                       int64_t* out, int64_t out_rs, int bnd, hipStream_t st) {
  hipLaunchKernelGGL(sel2_merge_kernel<PER>, dim3((unsigned)rows), dim3(kTopkThreads), 0, st, ws, ck, ci, crs, m, k,
                     out, out_rs, bnd);
}

// Both stages of a two-stage selection of k (chunks * k <= kSel2MaxCand) into out [rows] with row stride out_rs.
template <class KeyF>
void sel2_run(const KeyF& kf, int rows, int n, int k, const SelWs& ws, int cand_sel, int64_t* out, int64_t out_rs,
              hipStream_t st, bool bound = false) {
  const int bnd = bound ? 1 : 0;
  const int chunks = (n + kSel2Chunk - 1) / kSel2Chunk, m = chunks * k;
  hipLaunchKernelGGL(sel2_local_kernel<KeyF>, dim3((unsigned)chunks, (unsigned)rows), dim3(kTopkThreads), 0, st, kf, n,
                     k, ws, cand_sel);
  const uint32_t* ck = ws.ckey;
  const int* ci = ws.cidx;
  int64_t crs = m;
  int mm = m;
  if (k <= 512 && m > 16 * kTopkThreads) {
    // groups of whole chunks, at most 4 * kTopkThreads candidates each (at least 8 chunks: groups * k stays within
    // 65,536 / 8 + k <= kSel2C2). Measured on MI355X, top-256 of 32 x 1,048,576 (8 groups): 159.6 against 177.3 us
    // with the one-workgroup-per-row merge; RoCo's `pick` at 32 x 131,072 (2 groups) lost 3 % on the extra launch,
    // hence the group level only where the single merge would hold more than 16 candidates per lane.
    const int gslots = (4 * kTopkThreads / k) * k;
    const int groups = (m + gslots - 1) / gslots;
    hipLaunchKernelGGL(sel2_group_kernel<4>, dim3((unsigned)groups, (unsigned)rows), dim3(kTopkThreads), 0, st, ws, m,
                       k, gslots);
    ck = ws.c2key;
    ci = ws.c2idx;
    crs = kSel2C2;
    mm = groups * k;
  }
  if (mm <= 4 * kTopkThreads) sel2_merge_launch<4>(ws, ck, ci, crs, rows, mm, k, out, out_rs, bnd, st);
  else if (mm <= 16 * kTopkThreads) sel2_merge_launch<16>(ws, ck, ci, crs, rows, mm, k, out, out_rs, bnd, st);
  else if (mm <= 32 * kTopkThreads) sel2_merge_launch<32>(ws, ck, ci, crs, rows, mm, k, out, out_rs, bnd, st);
  else sel2_merge_launch<64>(ws, ck, ci, crs, rows, mm, k, out, out_rs, bnd, st);
}

// RoCo's output from its two two-stage selections: row r of out holds pick's `na` indices then recent's `nb`, each
// ascending; they are merged in place into one ascending list (an index in both written twice). One workgroup per
// row; both lists go through LDS as 32-bit indices (n <= 2^26), na + nb <= kRocoMergeMax. (Rows of more than 65,536
// keys have at least 9 chunks, so each list of the two-stage form holds at most 65,536 / 9 indices and the limit
// holds by itself; the host checks it anyway.)
constexpr int kRocoMergeMax = 16384;
__global__ void __launch_bounds__(256) roco_merge_kernel(int64_t* __restrict__ out, int na, int nb) {
  __shared__ int la[kRocoMergeMax];
  int* lb = la + na;
  int64_t* o = out + (int64_t)blockIdx.x * (na + nb);
  for (int i = threadIdx.x; i < na + nb; i += 256) la[i] = (int)o[i];
  __syncthreads();
  for (int i = threadIdx.x; i < na; i += 256) {  // position: i + the recent indices below it
    const int x = la[i];
    int lo = 0, hi = nb;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (lb[mid] < x) lo = mid + 1;
      else hi = mid;
    }
    o[i + lo] = x;
  }
  for (int j = threadIdx.x; j < nb; j += 256) {  // position: j + the pick indices at or below it
    const int x = lb[j];
    int lo = 0, hi = na;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (la[mid] <= x) lo = mid + 1;
      else hi = mid;
    }
    o[j + lo] = x;
  }
}

// One selection of k among the candidates (cand_sel's mask, or every key: kSelAll) into mask `sel`.
template <class KeyF>
void sel_run(const KeyF& kf, int rows, int n, const SelWs& ws, int sel, uint32_t k, int cand_sel, hipStream_t st) {
  const dim3 grid(ws.chunks, rows), block(kSelThreads);
  if (k == 0) {
    hipLaunchKernelGGL(sel_mark_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, k, cand_sel, 0, 0);
    return;
  }
  for (int ps = 0; ps < 2; ++ps)
    hipLaunchKernelGGL(sel_hist_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, ps, k, cand_sel);
  hipLaunchKernelGGL(sel_split_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, k, cand_sel);
  hipLaunchKernelGGL(sel_hist_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, 3, k, kSelPrefix);
  hipLaunchKernelGGL(sel_eqcount_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, k, kSelPrefix, 0);
  hipLaunchKernelGGL(sel_mark_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, k, kSelPrefix, 1, 0);
}

// RoCo's `other` after a two-stage `recent` that left its boundary (sel_bound): the mask of the n - recent smallest
// std keys, from one count of the keys equal to recent's K* and one marking pass.
template <class KeyF>
void sel_complement_run(const KeyF& kf, int rows, int n, const SelWs& ws, int sel, uint32_t k, hipStream_t st) {
  const dim3 grid(ws.chunks, rows), block(kSelThreads);
  hipLaunchKernelGGL(sel_eqcount_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, k, kSelAll, 1);
  hipLaunchKernelGGL(sel_mark_kernel<KeyF>, grid, block, 0, st, kf, n, ws, sel, k, kSelAll, 0, 1);
}

void sel_zero_hist(const SelWs& ws, int rows, hipStream_t st) {
  const int64_t count = (int64_t)rows * kSelNSel * 1024;
  const unsigned blocks = (unsigned)std::min<int64_t>(1024, (count + 255) / 256);
  hipLaunchKernelGGL(sel_zero_kernel, dim3(blocks), dim3(256), 0, st, ws.hist, count);
}

int sel_check_ws(const char* op, int64_t rows, int64_t n, void* workspace, int64_t workspace_bytes, SelWs* ws) {
  DGG_REQUIRE(rows < 65536, DGG_ERR_SHAPE, "%s: more than 65535 rows of over 65536 keys (got %lld rows)", op,
              (long long)rows);
  const int64_t need = sel_layout(rows, n, workspace, ws);
  DGG_REQUIRE(workspace != nullptr, DGG_ERR_NULL, "%s: rows of more than 65536 keys need a workspace", op);
  DGG_REQUIRE(workspace_bytes >= need, DGG_ERR_WORKSPACE, "%s: workspace of %lld bytes < required %lld", op,
              (long long)workspace_bytes, (long long)need);
  DGG_REQUIRE(((uintptr_t)workspace & 255u) == 0, DGG_ERR_ALIGN, "%s: workspace must be 256-byte aligned", op);
  return DGG_OK;
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

extern "C" int64_t dgg_select_workspace_bytes(int64_t rows, int64_t n) {
  if (rows < 0 || n < 0) return -1;
  if (n <= 65536) return 0;
  return sel_layout(rows, n, nullptr, nullptr);
}

extern "C" int dgg_topk_select_ws(const float* scores, int64_t rows, int64_t n, int64_t k, int largest,
                                  int64_t* out_idx, void* workspace, int64_t workspace_bytes, void* stream) {
  if (n <= 65536) return dgg_topk_select(scores, rows, n, k, largest, out_idx, stream);
  DGG_REQUIRE(n <= kSelMaxN, DGG_ERR_SHAPE, "topk_indices: n must be <= 2^26 (got %lld)", (long long)n);
  DGG_REQUIRE(rows >= 0, DGG_ERR_SHAPE, "topk_indices: bad row count %lld", (long long)rows);
  DGG_REQUIRE(k >= 1 && k <= n, DGG_ERR_SHAPE, "topk_indices: k must be in [1, n] (got k=%lld, n=%lld)",
              (long long)k, (long long)n);
  if (rows == 0) return DGG_OK;
  DGG_REQUIRE(scores && out_idx, DGG_ERR_NULL, "topk_indices: null pointer");
  SelWs ws;
  if (int rc = sel_check_ws("topk_indices", rows, n, workspace, workspace_bytes, &ws)) return rc;
  hipStream_t st = dgg::as_stream(stream);
  const KeyScores kf{scores, (int)n, largest ? 1 : 0};
  const int64_t chunks2 = (n + kSel2Chunk - 1) / kSel2Chunk;
  if (chunks2 * k <= kSel2MaxCand) {  // two stages: one read of the row
    sel2_run(kf, (int)rows, (int)n, (int)k, ws, kSelAll, out_idx, k, st);
    return dgg::check_launch("topk_indices");
  }
  sel_zero_hist(ws, (int)rows, st);
  sel_run(kf, (int)rows, (int)n, ws, 0, (uint32_t)k, kSelAll, st);
  hipLaunchKernelGGL(sel_emit_kernel, dim3(ws.chunks, (unsigned)rows), dim3(kSelThreads), 0, st, (int)n, ws, 0, -1,
                     out_idx, (int)k);
  return dgg::check_launch("topk_indices");
}

extern "C" int dgg_roco_select_ws(const float* score, const float* sq_score, int64_t rows, int64_t n, int64_t q_len,
                                  int64_t recent, int64_t budget, int64_t* out_idx, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (n <= 65536) return dgg_roco_select(score, sq_score, rows, n, q_len, recent, budget, out_idx, stream);
  DGG_REQUIRE(n <= kSelMaxN, DGG_ERR_SHAPE, "roco_select: n must be <= 2^26 (got %lld)", (long long)n);
  DGG_REQUIRE(rows >= 0, DGG_ERR_SHAPE, "roco_select: bad row count %lld", (long long)rows);
  DGG_REQUIRE(q_len >= 1 && q_len <= (1ll << 24), DGG_ERR_SHAPE, "roco_select: q_len must be in [1, 2^24] (got %lld)",
              (long long)q_len);
  DGG_REQUIRE(recent >= 0 && recent <= n, DGG_ERR_SHAPE, "roco_select: recent must be in [0, n] (got %lld, n=%lld)",
              (long long)recent, (long long)n);
  DGG_REQUIRE(budget >= 0 && budget <= n - recent, DGG_ERR_SHAPE,
              "roco_select: budget must be in [0, n - recent] (got %lld, n=%lld, recent=%lld)", (long long)budget,
              (long long)n, (long long)recent);
  if (rows == 0 || budget + recent == 0) return DGG_OK;
  DGG_REQUIRE(score && sq_score && out_idx, DGG_ERR_NULL, "roco_select: null pointer");
  SelWs ws;
  if (int rc = sel_check_ws("roco_select", rows, n, workspace, workspace_bytes, &ws)) return rc;
  hipStream_t st = dgg::as_stream(stream);
  const float rcp = 1.0f / (float)q_len;  // torch's reciprocal of the Python divisor, in fp32
  const int R = (int)rows, N = (int)n;
  const int64_t chunks2 = (n + kSel2Chunk - 1) / kSel2Chunk;
  if (chunks2 * std::max(recent, budget) <= kSel2MaxCand && budget + recent <= kRocoMergeMax) {
    // recent and pick in two stages (pick among other's mask), other from recent's boundary; the two index lists
    // are written to out's rows (pick first) and merged in place
    const int64_t rs = budget + recent;
    if (recent > 0)  // roco.py:56, leaving its boundary for `other`
      sel2_run(KeyStd{score, sq_score, N, rcp, 0}, R, N, (int)recent, ws, kSelAll, out_idx + budget, rs, st, true);
    if (budget > 0) {
      if (recent > 0) {  // roco.py:55 from recent's boundary, then roco.py:57-58 among its keys
        sel_complement_run(KeyStd{score, sq_score, N, rcp, 1}, R, N, ws, 1, (uint32_t)(n - recent), st);
        sel2_run(KeyMean{score, N, rcp}, R, N, (int)budget, ws, 1, out_idx, rs, st);
      } else {  // `other` is every key
        sel2_run(KeyMean{score, N, rcp}, R, N, (int)budget, ws, kSelAll, out_idx, rs, st);
      }
    }
    if (budget > 0 && recent > 0)
      hipLaunchKernelGGL(roco_merge_kernel, dim3((unsigned)rows), dim3(256), 0, st, out_idx, (int)budget, (int)recent);
    return dgg::check_launch("roco_select");
  }
  sel_zero_hist(ws, R, st);
  sel_run(KeyStd{score, sq_score, N, rcp, 0}, R, N, ws, 0, (uint32_t)recent, kSelAll, st);      // roco.py:56
  sel_run(KeyStd{score, sq_score, N, rcp, 1}, R, N, ws, 1, (uint32_t)(n - recent), kSelAll, st);  // roco.py:55
  sel_run(KeyMean{score, N, rcp}, R, N, ws, 2, (uint32_t)budget, 1, st);                   // roco.py:57-58
  hipLaunchKernelGGL(sel_emit_kernel, dim3(ws.chunks, (unsigned)rows), dim3(kSelThreads), 0, st, N, ws, 2, 0, out_idx,
                     (int)(budget + recent));
  return dgg::check_launch("roco_select");
}
