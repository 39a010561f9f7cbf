// kbh_w4a16_gemm_noalloc: the W4A16 GEMM of kbh_w4a16_gemm with its split-K partial sums in a
// fixed per-GPU array of this library instead of caller buffers (no counterpart in the reference;
// for callers that cannot allocate device memory or pass a workspace).
//
// The array lives in this translation unit on purpose. Each .hip file is its own code object,
// loaded onto a GPU when first needed there, and a __device__ variable is reserved with its
// code object: kept in w4a16.hip, the 64 MiB were reserved on every GPU that ran any W4A16 call
// (measured: +68 MiB at the first kbh_w4a16_gemm call). Here nothing but the symbol lookup of
// the first no-alloc call on a GPU loads it, so only its users pay.
#include <atomic>
#include <mutex>

#include "kbh_common.h"

namespace kbh {
// The scratch need of the path a W4A16 call takes (defined with the kernels in w4a16.hip).
size_t w4a16_path_bytes(int M, int N, int K, int group);

namespace {

// Each GPU the library runs on holds its own copy, at its own address, until the process ends.
// In host code the name is only a stand-in for the symbol: the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) uint8_t scratch[KBH_W4A16_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first call there).
int noalloc_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_last_hip_error((int)e);
    return KBH_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) return KBH_ERR_LAUNCH;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        set_last_hip_error((int)e);
        return KBH_ERR_LAUNCH;
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return KBH_OK;
}

}  // namespace
}  // namespace kbh

// Shapes whose path needs more than the array return KBH_ERR_SCRATCH_LIMIT before any HIP call.
extern "C" int kbh_w4a16_gemm_noalloc(const void* x, const int32_t* qweight, const void* scales,
                                      const void* zeros, void* y, int M, int N, int K, int group,
                                      int dtype, void* stream) {
  using namespace kbh;
  if (!x || !qweight || !scales || !zeros || !y) return KBH_ERR_NULL;
  if (dtype != KBH_F16 && dtype != KBH_BF16) return KBH_ERR_DTYPE;
  if (M < 1 || N < 128 || K < 32 || (N % 128) != 0 || (K % 32) != 0) return KBH_ERR_SHAPE;
  if (group != 32 && group != 64 && group != 128 && group != 256) return KBH_ERR_SHAPE;
  if (K % group != 0) return KBH_ERR_SHAPE;
  const size_t need = w4a16_path_bytes(M, N, K, group);
  if (need > KBH_W4A16_NOALLOC_SCRATCH_BYTES) return KBH_ERR_SCRATCH_LIMIT;
  void* p = nullptr;
  const int st = noalloc_scratch(&p);
  if (st != KBH_OK) return st;
  // The path uses one of the two buffers, so both may name the array.
  return kbh_w4a16_gemm(x, qweight, scales, zeros, y, p, KBH_W4A16_NOALLOC_SCRATCH_BYTES, p,
                        KBH_W4A16_NOALLOC_SCRATCH_BYTES, M, N, K, group, dtype, stream);
}
