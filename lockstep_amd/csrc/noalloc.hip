// The allocation-free dense contract linear: lsk_w8a8_matmul with its workspace (the quantised
// rows and their scales) in a fixed device array of this library instead of caller memory, for
// callers that cannot allocate (code under graph capture, tight serving loops, harnesses that
// forbid hipMalloc).
#include <mutex>

#include "lsk_common.h"

extern "C" int64_t lsk_w8a8_matmul_workspace(int64_t M, int64_t K);
extern "C" int lsk_w8a8_matmul(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                               int64_t ldw, int64_t N, const float* ws, const float* bias, int order, void* out,
                               int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream);

// 16 MiB per GPU, held until the process ends: M rows of width K fit when
// M * ceil16(K) (rounded up to 256) + 4 * M (rounded up to 256) <= 16 MiB, e.g. every decode batch
// of the configs' projections and 2048 prefill rows at K = 4096.
constexpr int64_t kScratchBytes = 16ll << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch` on each device, looked up once
std::mutex g_scratch_mu;

// The current device's copy of `scratch`.  The array's name is a host-side stand-in, never a
// device address: the address comes from hipGetSymbolAddress, called once per device with that
// device current.
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    lsk::set_error("lsk_w8a8_matmul_noalloc: no usable current device (%d)", dev);
    return LSK_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      lsk::set_error("lsk_w8a8_matmul_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                     hipGetErrorString(e));
      return LSK_ERR_HIP;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return LSK_OK;
}

}  // namespace

extern "C" int lsk_w8a8_matmul_noalloc(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                       const int8_t* w, int64_t ldw, int64_t N, const float* ws, const float* bias,
                                       int order, void* out, int out_dtype, int64_t ldo, void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_w8a8_matmul_noalloc: negative size");
  if (M > 0 && N > 0) {
    const int64_t need = lsk_w8a8_matmul_workspace(M, K);
    LSK_REQUIRE(need <= kScratchBytes,
                "lsk_w8a8_matmul_noalloc: M=%lld rows of K=%lld need %lld bytes of scratch, above its maximum of "
                "%lld bytes (call lsk_w8a8_matmul with a workspace instead)",
                (long long)M, (long long)K, (long long)need, (long long)kScratchBytes);
  }
  void* buf = nullptr;
  if (M > 0 && N > 0) {
    const int rc = scratch_of_current_device(&buf);
    if (rc) return rc;
  }
  return lsk_w8a8_matmul(x, x_dtype, ldx, M, K, w, ldw, N, ws, bias, order, out, out_dtype, ldo, buf, kScratchBytes,
                         stream);
}
