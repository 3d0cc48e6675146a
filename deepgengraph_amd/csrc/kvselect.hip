// KV-cache selection ops around the column-score kernels: SnapKV's pooling of the column sums and the gather
// of the selected key/value rows into the compacted cache.
//
// Both are HBM-bound and tiny next to attention: one thread per output float (pooling) or per 16-byte chunk of
// a selected row (gather), 256 threads per workgroup, grid-stride loops.
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
