// Shared device/host helpers for the gfx950 kernels behind include/dgg.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "../../include/dgg.h"

// ----------------------------------------------------------------------------------------------
// Host side: thread-local error message + status helpers.
// ----------------------------------------------------------------------------------------------
namespace dgg {

int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int dtype_size(int dtype) { return dtype == DGG_F32 ? 4 : 2; }
inline bool valid_dtype(int dtype) { return dtype == DGG_F32 || dtype == DGG_F16 || dtype == DGG_BF16; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Decode (decode.hip): validates the arguments of a dgg_attn_decode call and launches it with the split partials in
// `workspace`. With resolve_ws (the allocation-free entry point, decode_noalloc.hip), workspace_bytes is the size of
// a fixed buffer that resolve_ws supplies once the arguments are valid.
int decode_launch(const char* op, const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                  int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                  const int64_t* strides, int64_t splits, float scale, int dtype, void* stream,
                  int (*resolve_ws)(const char* op, void* stream, void** ws));

// Split-KV attention (splitkv.hip): validates the arguments of a dgg_attn_splitkv call and launches it with the split
// partials in `workspace` (resolve_ws as for decode_launch). Grouped-query decode calls run through it.
int splitkv_launch(const char* op, const void* q, const void* k, const void* v, void* o, float* lse, void* workspace,
                   int64_t workspace_bytes, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D,
                   const int64_t* strides, int64_t splits, float scale, float softcap, int64_t window, uint32_t flags,
                   int dtype, void* stream, int (*resolve_ws)(const char* op, void* stream, void** ws));

}  // namespace dgg

#define DGG_REQUIRE(cond, code, ...)            \
  do {                                          \
    if (!(cond)) return dgg::set_error(code, __VA_ARGS__); \
  } while (0)

// ----------------------------------------------------------------------------------------------
// Device side: vector types and conversions.
// ----------------------------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

// Storage tags: kernels are templated on one of these. `vec8` is the 16-byte vector of 8 elements.
struct F16 {
  typedef _Float16 scalar;
  typedef f16x8 vec8;
  typedef f16x4 vec4;
};
struct BF16 {
  typedef __bf16 scalar;
  typedef bf16x8 vec8;
  typedef bf16x4 vec4;
};
struct F32 {
  typedef float scalar;
};

// Round-to-nearest-even conversions (the compiler lowers these to v_cvt_* for gfx950).
template <typename S>
__device__ __forceinline__ S to_s(float x) {
  return static_cast<S>(x);
}
template <typename S>
__device__ __forceinline__ float to_f(S x) {
  return static_cast<float>(x);
}

__device__ __forceinline__ f32x8 to_f32x8(f16x8 v) { return __builtin_convertvector(v, f32x8); }
__device__ __forceinline__ f32x8 to_f32x8(bf16x8 v) { return __builtin_convertvector(v, f32x8); }
template <typename V>
__device__ __forceinline__ V from_f32x8(f32x8 v) {
  return __builtin_convertvector(v, V);
}

// 16-byte global loads/stores of 8 elements.
template <typename V>
__device__ __forceinline__ V ld16(const void* p) {
  return *reinterpret_cast<const V*>(p);
}
template <typename V>
__device__ __forceinline__ void st16(void* p, V v) {
  *reinterpret_cast<V*>(p) = v;
}
// The same with the non-temporal hint, for data a kernel reads or writes once (a streamed row, an output nobody
// re-reads in the same kernel).
template <typename V>
__device__ __forceinline__ V ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
}
template <typename V>
__device__ __forceinline__ void st16_nt(void* p, V v) {
  __builtin_nontemporal_store(v, reinterpret_cast<V*>(p));
}

// Pointers in the global address space (loads through them are global_load_*, never flat_load_*).
typedef const char __attribute__((address_space(1)))* gptr;
template <typename V>
__device__ __forceinline__ V ldg16(gptr p) {
  return *reinterpret_cast<const V __attribute__((address_space(1)))*>(p);
}
__device__ __forceinline__ gptr to_gptr(const void* p) { return (gptr)(reinterpret_cast<uintptr_t>(p)); }

// Wave64 reductions.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// exp2 of a value known to be <= a few hundred: the hardware v_exp_f32 (handles -inf -> 0).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
