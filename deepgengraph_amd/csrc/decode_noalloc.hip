// Allocation-free decode (dgg_attn_decode_noalloc): dgg_attn_decode with the split partials in `scratch`, a
// file-scope device array of kDecodeScratchBytes, instead of a caller-provided workspace.
//
// The array sits in this file's code object alone. The library is built without relocatable device code, so each
// source file is its own code object, which the HIP runtime loads onto a device the first time something in it is
// used there. A process that never calls dgg_attn_decode_noalloc on a device therefore never takes the 96 MiB on it;
// one that does holds it on that device until the process ends.
//
// Host code never passes the array's name to a kernel (on the host it is only a stand-in for the symbol): its
// device address is looked up once per device with hipGetSymbolAddress and cached. The partial kernels write every
// partial entry before the merge reads it, so nothing needs clearing between calls; calls that overlap on one GPU
// share the array and race.
#include <mutex>

#include "common.h"

namespace {

constexpr int64_t kDecodeScratchBytes = 96ll << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's `scratch`, for the device the stream runs on (which must be current).
int device_scratch(const char* op, void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  DGG_REQUIRE(e == hipSuccess, DGG_ERR_LAUNCH, "%s: hipGetDevice failed: %s", op, hipGetErrorString(e));
  DGG_REQUIRE(dev >= 0 && dev < kMaxDevices, DGG_ERR_LAUNCH, "%s: device %d out of range", op, dev);
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(dgg::as_stream(stream), &sdev);
    DGG_REQUIRE(e == hipSuccess, DGG_ERR_LAUNCH, "%s: hipStreamGetDevice failed: %s", op, hipGetErrorString(e));
    DGG_REQUIRE(sdev == dev, DGG_ERR_LAUNCH, "%s: the stream belongs to device %d but device %d is current", op, sdev,
                dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    DGG_REQUIRE(e == hipSuccess && ptr != nullptr, DGG_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", op,
                hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return DGG_OK;
}

}  // namespace

extern "C" int dgg_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                                       int64_t Hq, int64_t Hkv, int64_t L, int64_t D, const int64_t* strides,
                                       int64_t splits, float scale, int dtype, void* stream) {
  return dgg::decode_launch("attn_decode_noalloc", q, k, v, o, lse, nullptr, kDecodeScratchBytes, B, Hq, Hkv, L, D,
                            strides, splits, scale, dtype, stream, device_scratch);
}
