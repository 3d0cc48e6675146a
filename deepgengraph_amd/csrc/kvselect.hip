// KV-cache selection ops around the column-score kernels: SnapKV's pooling of the column sums, the gather of the
// selected key/value rows into the compacted cache, and Corm's nonzero (the coordinates of the selected keys).
//
// All are HBM-bound and tiny next to attention: one thread per output float (pooling) or per 16-byte chunk of
// a selected row (gather), 256 threads per workgroup, grid-stride loops; nonzero is a three-launch stream
// compaction (row counts, an exclusive scan over the rows, ordered writes).
#include <algorithm>

#include "common.h"

namespace {

constexpr int kThreads = 256;

// out[r][j] = sum_{t = j-h}^{j+h} in[r][t] / ks (zero outside [0, n)), h = ks / 2: F.avg_pool1d with
// padding ks // 2, stride 1 and the default count_include_pad (snapkv.py:38).
__global__ void __launch_bounds__(kThreads) avg_pool1d_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                              int64_t rows, int64_t n, int ks) {
  const int h = ks / 2;
  const float inv = 1.0f / (float)ks;
  const int64_t total = rows * n;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total; e += (int64_t)gridDim.x * kThreads) {
    const int64_t r = e / n, j = e - r * n;
    const float* row = in + r * n;
    float acc = 0.f;
    for (int t = -h; t <= h; ++t) {
      const int64_t c = j + t;
      if (c >= 0 && c < n) acc += row[c];
    }
    out[e] = acc * inv;
  }
}

// out[b][s][i][h][:] = (s == 0 ? k : v)[b][idx[b][h][i]][h][:] (models/h2o.py:53-56). Rows are row_b bytes,
// copied as 16-byte chunks; an index outside [0, S) yields a zero row (the cache is never read out of bounds).
struct GatherParams {
  const char* k;
  const char* v;
  const int64_t* idx;
  char* out;
  int64_t k_sb, k_ss, k_sh;  // byte strides
  int64_t v_sb, v_ss, v_sh;
  int B, S, Hkv, n_sel, chunks;  // chunks = row bytes / 16
};

// ---- nonzero (models/corm.py:53: torch.nonzero(corm_score)) ----------------------------------------------
// The input is viewed as [rows, n] bytes (row-major); a nonzero element at flat index f is written as its ndim
// coordinates (f decomposed by dims, last dimension fastest) at position (nonzeros before row) + (rank in row),
// which is torch.nonzero's row-major order.
constexpr int kMaxNonzeroDims = 8;
struct NonzeroParams {
  const uint8_t* in;
  int64_t rows, n;
  int64_t* counts;   // [rows + 1]: per-row counts, then (after the scan) exclusive offsets and the total
  int64_t* coords;   // [max_out, ndim]
  int64_t* total;    // device int64: number of nonzeros
  int64_t max_out;
  int ndim;
  int64_t dims[kMaxNonzeroDims];
};

__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  int64_t t = 0;
  for (int i = 0; i < (int)blockDim.x / 64; ++i) t += red[i];
  __syncthreads();
  return t;
}

__global__ void __launch_bounds__(kThreads) nonzero_count_kernel(NonzeroParams p) {
  __shared__ int64_t red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const uint8_t* x = p.in + row * p.n;
  int64_t c = 0;
  for (int64_t j = threadIdx.x; j < p.n; j += kThreads) c += x[j] != 0;
  c = block_sum_i64(c, red);
  if (threadIdx.x == 0) p.counts[row] = c;
}

// One workgroup: exclusive scan of the row counts in place, total into counts[rows] and *total.
__global__ void __launch_bounds__(1024) nonzero_scan_kernel(NonzeroParams p) {
  __shared__ int64_t wsum[16];
  int64_t carry = 0;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int64_t base = 0; base < p.rows; base += 1024) {
    const int64_t r = base + threadIdx.x;
    const int64_t v = r < p.rows ? p.counts[r] : 0;
    int64_t incl = v;  // inclusive scan within the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t u = __shfl_up(incl, off, 64);
      if (lane >= off) incl += u;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    int64_t before = 0, chunk = 0;
    for (int i = 0; i < 16; ++i) {
      if (i < w) before += wsum[i];
      chunk += wsum[i];
    }
    if (r < p.rows) p.counts[r] = carry + before + incl - v;
    carry += chunk;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    p.counts[p.rows] = carry;
    *p.total = carry;
  }
}

__global__ void __launch_bounds__(kThreads) nonzero_write_kernel(NonzeroParams p) {
  __shared__ int wcount[kThreads / 64];
  const int64_t row = blockIdx.x;
  const uint8_t* x = p.in + row * p.n;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t pos0 = p.counts[row];
  for (int64_t base = 0; base < p.n; base += kThreads) {
    const int64_t j = base + threadIdx.x;
    const bool f = j < p.n && x[j] != 0;
    const uint64_t ball = __ballot(f);
    const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(ball >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ball, 0));
    if (lane == 0) wcount[w] = __popcll(ball);
    __syncthreads();
    int before = 0, chunk = 0;
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) {
      if (i < w) before += wcount[i];
      chunk += wcount[i];
    }
    const int64_t pos = pos0 + before + rank;
    if (f && pos < p.max_out) {
      int64_t flat = row * p.n + j;
      int64_t* dst = p.coords + pos * p.ndim;
      for (int d = p.ndim - 1; d >= 0; --d) {
        const int64_t q = flat / p.dims[d];
        dst[d] = flat - q * p.dims[d];
        flat = q;
      }
    }
    pos0 += chunk;
    __syncthreads();
  }
}

__global__ void __launch_bounds__(64) nonzero_zero_kernel(int64_t* total) {
  if (threadIdx.x == 0) *total = 0;
}

__global__ void __launch_bounds__(kThreads) kv_gather_kernel(GatherParams p) {
  const int64_t total = (int64_t)p.B * 2 * p.n_sel * p.Hkv * p.chunks;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total; e += (int64_t)gridDim.x * kThreads) {
    // e enumerates the output [B, 2, n_sel, Hkv, chunks] in order, so the stores are contiguous.
    int64_t t = e;
    const int c = (int)(t % p.chunks);
    t /= p.chunks;
    const int h = (int)(t % p.Hkv);
    t /= p.Hkv;
    const int i = (int)(t % p.n_sel);
    t /= p.n_sel;
    const int which = (int)(t % 2);
    const int b = (int)(t / 2);
    const int64_t row = p.idx[((int64_t)b * p.Hkv + h) * p.n_sel + i];
    u16x8 val = {};
    if (row >= 0 && row < p.S) {
      const char* src = which == 0 ? p.k + b * p.k_sb + row * p.k_ss + h * p.k_sh
                                   : p.v + b * p.v_sb + row * p.v_ss + h * p.v_sh;
      val = ld16<u16x8>(src + 16 * c);
    }
    st16<u16x8>(p.out + 16 * e, val);
  }
}

unsigned grid_for(int64_t total) {
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  return (unsigned)std::min<int64_t>(blocks, 256 * 64);
}

}  // namespace

extern "C" int dgg_avg_pool1d(const float* in, float* out, int64_t rows, int64_t n, int64_t kernel_size, void* stream) {
  DGG_REQUIRE(rows >= 0 && n >= 0 && rows * n < (1ll << 40), DGG_ERR_SHAPE, "avg_pool1d: bad shape [%lld, %lld]",
              (long long)rows, (long long)n);
  DGG_REQUIRE(kernel_size >= 1 && kernel_size % 2 == 1 && kernel_size < 4096, DGG_ERR_UNSUPPORTED,
              "avg_pool1d: kernel_size must be odd and in [1, 4095] (got %lld)", (long long)kernel_size);
  if (rows == 0 || n == 0) return DGG_OK;
  DGG_REQUIRE(in && out, DGG_ERR_NULL, "avg_pool1d: null pointer");
  DGG_REQUIRE(in != out, DGG_ERR_SHAPE, "avg_pool1d: out must not alias in");
  hipLaunchKernelGGL(avg_pool1d_kernel, dim3(grid_for(rows * n)), dim3(kThreads), 0, dgg::as_stream(stream), in, out,
                     rows, n, (int)kernel_size);
  return dgg::check_launch("avg_pool1d");
}

extern "C" int dgg_kv_gather(const void* k, const void* v, const int64_t* indices, void* out, int64_t B, int64_t S,
                             int64_t Hkv, int64_t D, int64_t n_sel, const int64_t* strides, int dtype, void* stream) {
  const char* op = "kv_gather";
  DGG_REQUIRE(dgg::valid_dtype(dtype), DGG_ERR_DTYPE, "%s: bad dtype code %d", op, dtype);
  DGG_REQUIRE(B >= 0 && S >= 0 && Hkv >= 1 && D >= 1 && n_sel >= 0 && B < (1 << 20) && S < (1ll << 31) &&
                  Hkv < (1 << 16) && n_sel < (1ll << 31),
              DGG_ERR_SHAPE, "%s: bad sizes", op);
  const int64_t row_b = D * dgg::dtype_size(dtype);
  DGG_REQUIRE(row_b % 16 == 0, DGG_ERR_SHAPE, "%s: a row of D elements must be a multiple of 16 bytes", op);
  DGG_REQUIRE(strides != nullptr, DGG_ERR_NULL, "%s: strides is NULL", op);
  if (B == 0 || n_sel == 0) return DGG_OK;
  DGG_REQUIRE(k && v && indices && out, DGG_ERR_NULL, "%s: null pointer", op);
  const int64_t es = dgg::dtype_size(dtype);
  for (int i = 0; i < 6; ++i)
    DGG_REQUIRE(strides[i] >= 0 && (strides[i] * es) % 16 == 0, DGG_ERR_STRIDE,
                "%s: stride[%d] = %lld must keep rows 16-byte aligned", op, i, (long long)strides[i]);
  DGG_REQUIRE(dgg::aligned16(k) && dgg::aligned16(v) && dgg::aligned16(out), DGG_ERR_ALIGN,
              "%s: k, v and out must be 16-byte aligned", op);
  GatherParams p{};
  p.k = static_cast<const char*>(k);
  p.v = static_cast<const char*>(v);
  p.idx = indices;
  p.out = static_cast<char*>(out);
  p.k_sb = strides[0] * es; p.k_ss = strides[1] * es; p.k_sh = strides[2] * es;
  p.v_sb = strides[3] * es; p.v_ss = strides[4] * es; p.v_sh = strides[5] * es;
  p.B = (int)B;
  p.S = (int)S;
  p.Hkv = (int)Hkv;
  p.n_sel = (int)n_sel;
  p.chunks = (int)(row_b / 16);
  hipLaunchKernelGGL(kv_gather_kernel, dim3(grid_for(B * 2 * n_sel * Hkv * p.chunks)), dim3(kThreads), 0,
                     dgg::as_stream(stream), p);
  return dgg::check_launch(op);
}

extern "C" int64_t dgg_nonzero_workspace_bytes(int64_t rows) { return rows < 0 ? -1 : (rows + 1) * 8; }

extern "C" int dgg_nonzero(const uint8_t* in, int ndim, const int64_t* dims, int64_t* coords, int64_t max_out,
                           int64_t* total, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* op = "nonzero";
  DGG_REQUIRE(ndim >= 1 && ndim <= kMaxNonzeroDims, DGG_ERR_SHAPE, "%s: ndim %d not in [1, %d]", op, ndim,
              kMaxNonzeroDims);
  DGG_REQUIRE(dims != nullptr && total != nullptr, DGG_ERR_NULL, "%s: null dims / total", op);
  int64_t numel = 1;
  for (int d = 0; d < ndim; ++d) {
    DGG_REQUIRE(dims[d] >= 0 && dims[d] < (1ll << 40), DGG_ERR_SHAPE, "%s: dims[%d] invalid", op, d);
    numel *= dims[d];
    DGG_REQUIRE(numel < (1ll << 40), DGG_ERR_SHAPE, "%s: too many elements", op);
  }
  const int64_t n = dims[ndim - 1];
  const int64_t rows = n == 0 ? 0 : numel / n;
  DGG_REQUIRE(rows < (1ll << 31), DGG_ERR_SHAPE, "%s: too many rows", op);
  DGG_REQUIRE(max_out >= 0, DGG_ERR_SHAPE, "%s: max_out must be >= 0", op);
  hipStream_t st = dgg::as_stream(stream);
  if (rows == 0) {  // an empty input: total = 0 (a kernel rather than a memset node, so graph capture stays safe)
    hipLaunchKernelGGL(nonzero_zero_kernel, dim3(1), dim3(64), 0, st, total);
    return dgg::check_launch(op);
  }
  DGG_REQUIRE(in != nullptr && workspace != nullptr, DGG_ERR_NULL, "%s: null input / workspace", op);
  DGG_REQUIRE(max_out == 0 || coords != nullptr, DGG_ERR_NULL, "%s: null coords", op);
  DGG_REQUIRE(workspace_bytes >= dgg_nonzero_workspace_bytes(rows), DGG_ERR_SHAPE,
              "%s: workspace of %lld bytes < %lld", op, (long long)workspace_bytes,
              (long long)dgg_nonzero_workspace_bytes(rows));
  DGG_REQUIRE(((uintptr_t)workspace & 7u) == 0 && ((uintptr_t)total & 7u) == 0 && ((uintptr_t)coords & 7u) == 0,
              DGG_ERR_ALIGN, "%s: workspace, total and coords must be 8-byte aligned", op);
  NonzeroParams p{};
  p.in = in;
  p.rows = rows;
  p.n = n;
  p.counts = static_cast<int64_t*>(workspace);
  p.coords = coords;
  p.total = total;
  p.max_out = max_out;
  p.ndim = ndim;
  for (int d = 0; d < ndim; ++d) p.dims[d] = dims[d];
  hipLaunchKernelGGL(nonzero_count_kernel, dim3((unsigned)rows), dim3(kThreads), 0, st, p);
  hipLaunchKernelGGL(nonzero_scan_kernel, dim3(1), dim3(1024), 0, st, p);
  hipLaunchKernelGGL(nonzero_write_kernel, dim3((unsigned)rows), dim3(kThreads), 0, st, p);
  return dgg::check_launch(op);
}
