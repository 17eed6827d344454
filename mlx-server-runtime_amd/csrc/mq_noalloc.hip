// mq_quantized_matmul_noalloc: mq_quantized_matmul_ws whose split-K partial
// sums live in a fixed device array of this library instead of a caller
// workspace, for callers that cannot allocate (code under HIP graph capture,
// serving loops that forbid hipMalloc).  Declared in include/mq.h.
//
// The array `scratch` below is a device global: every GPU the library runs on
// holds its own copy (kScratchBytes) until the process ends.  Host code never
// passes `scratch` itself (its host-side name is not a device address): a
// call with work to do on a device first resolves that device's copy with
// hipGetSymbolAddress, with the device current, and keeps the pointer once
// the lookup has succeeded (a failed lookup is returned and retried by the
// next call); every later call uses the resolved pointer.  The lookup is a
// runtime query, not stream work: callers that capture this entry point in a
// HIP graph make one eager call on the device first, so that no lookup
// happens during capture.  Calls on one GPU share its copy, so calls that
// overlap on one GPU (different streams, no ordering between them) race;
// calls ordered on one stream do not.  Nothing in the array needs clearing:
// each split writes all of its partial sums before the reduce reads them.
#include <mutex>

#include "../../include/mq.h"
#include "mq_internal.h"

namespace {

constexpr size_t kScratchBytes = MQ_NOALLOC_SCRATCH_BYTES;  // 16 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu[kMaxDevices];
void* g_scratch[kMaxDevices];  // non-null once resolved on that device

// Device address of `scratch` on device `dev`: resolved on the first call
// that succeeds, then reused.
hipError_t scratch_on(int dev, void** out) {
  std::lock_guard<std::mutex> lock(g_mu[dev]);
  if (g_scratch[dev]) {
    *out = g_scratch[dev];
    return hipSuccess;
  }
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
  void* p = nullptr;
  if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (cur >= 0 && cur != dev) {
    const hipError_t r = hipSetDevice(cur);
    if (e == hipSuccess) e = r;
  }
  if (e == hipSuccess && !p) e = hipErrorInvalidSymbol;
  if (e == hipSuccess) g_scratch[dev] = p;
  *out = p;
  return e;
}

}  // namespace

extern "C" int mq_quantized_matmul_noalloc(const mq_bf16* x, const uint32_t* wq,
                                           const mq_bf16* scales, const mq_bf16* biases,
                                           const mq_bf16* bias_vec, mq_bf16* y, int64_t M,
                                           int64_t N, int64_t K, int group_size, int bits,
                                           int transpose, hipStream_t stream) {
  size_t need = mq_quantized_matmul_workspace(M, N, K, group_size, bits);
  // a stream-K plan that does not fit the array runs every tile whole
  if (need > kScratchBytes && mq::qmm_workspace_optional(M, N, K, group_size, bits)) need = 0;
  if (need > kScratchBytes) {
    char msg[256];
    snprintf(msg, sizeof(msg),
             "[quantized_matmul_noalloc] M=%lld, N=%lld, K=%lld needs %zu bytes of scratch "
             "(split-K partial sums; at 2/3/5/6 bits also the codes repacked to 8 bits); this "
             "entry point holds %zu per GPU (use mq_quantized_matmul_ws with a caller "
             "workspace).",
             (long long)M, (long long)N, (long long)K, need, kScratchBytes);
    return mq::set_last_error(MQ_ERR_INVALID, msg);
  }
  void* ws = nullptr;
  // Resolved whenever the call has work, even where this plan needs no
  // scratch, so that one eager call of any size settles the lookup.
  if (M > 0 && N > 0 && K > 0) {
    int dev = -1;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices)) e = hipErrorInvalidDevice;
    if (e == hipSuccess) e = scratch_on(dev, &ws);
    if (e != hipSuccess) {
      char msg[192];
      snprintf(msg, sizeof(msg), "[quantized_matmul_noalloc] device scratch unavailable: %s",
               hipGetErrorString(e));
      return mq::set_last_error(MQ_ERR_HIP, msg);
    }
  }
  return mq_quantized_matmul_ws(x, wq, scales, biases, bias_vec, y, M, N, K, group_size, bits,
                                transpose, need > 0 ? ws : nullptr, need, stream);
}
