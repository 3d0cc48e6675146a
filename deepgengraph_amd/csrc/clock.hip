// Shader-clock probe for the benchmark: one lane reads the 64-bit cycle counter (s_memtime) and the constant
// 100 MHz real-time counter (s_memrealtime) around a spin of `ticks` real-time ticks; the ratio of the two deltas
// is the shader clock at that moment in units of 100 MHz. The spin ends once the real-time counter has advanced by
// `ticks` (bounded by the host to 1..10^6 ticks, i.e. at most 10 ms).
#include "common.h"

namespace {

__global__ void clock_probe_kernel(unsigned long long* out, unsigned long long ticks) {
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  unsigned long long r1 = r0;
  while (r1 - r0 < ticks) r1 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  out[0] = c1 - c0;
  out[1] = r1 - r0;
}

}  // namespace

extern "C" int dgg_clock_probe(unsigned long long* out, int64_t ticks, void* stream) {
  DGG_REQUIRE(out != nullptr, DGG_ERR_NULL, "clock_probe: null output");
  DGG_REQUIRE(((uintptr_t)out & 7u) == 0, DGG_ERR_ALIGN, "clock_probe: output must be 8-byte aligned");
  DGG_REQUIRE(ticks >= 1 && ticks <= 1000000, DGG_ERR_SHAPE, "clock_probe: ticks must be in [1, 10^6] (got %lld)",
              (long long)ticks);
  hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(1), 0, dgg::as_stream(stream), out,
                     (unsigned long long)ticks);
  return dgg::check_launch("clock_probe");
}
