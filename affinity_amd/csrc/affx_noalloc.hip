// The decode entry for callers that cannot allocate (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc): affx_expert_ffn_decode with its workspace in a
// file-scope device array instead of a caller buffer. Nothing here allocates.
//
// The array is one per GPU (each device holds its own copy of the code object's globals) and
// lives until the process ends. Host code never uses the array's name as an address: the
// per-device address comes from hipGetSymbolAddress, once per device with that device current.
// Calls on one GPU share its array: two calls that overlap on one GPU (different streams,
// different threads) race on it. The decode leaves its sync run zero after every launch and
// rewrites everything else it reads, so consecutive calls need no clearing; the set-up zeroes the
// array once (a fill kernel on the caller's stream: legal under graph capture, where a memset
// node is not used).
#include <mutex>

#include "affx_common.h"

namespace affx {

// The largest decode it serves: m_tokens <= 8, m_tokens * top_k <= 64, hidden <= 4096,
// inter <= 2048 (V4-Flash: 6 routes per token, so up to 8 tokens).
constexpr uint32_t kNaMaxTok = 8, kNaMaxRoutes = 64, kNaMaxHidden = 4096, kNaMaxInter = 2048;
constexpr uint64_t kNaScratchBytes = 3u * 1024u * 1024u + 256u * 1024u;  // 3.25 MiB

static __device__ __align__(256) uint8_t scratch[kNaScratchBytes];

__global__ void __launch_bounds__(256) noalloc_zero_kernel(uint4* __restrict__ p, uint64_t n16) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * 256)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

}  // namespace affx

using namespace affx;

namespace {

constexpr int kNaMaxDev = 64;
std::mutex g_na_mu;
uint8_t* g_na_ptr[kNaMaxDev];  // device address of `scratch` on each device (null: not set up)

// Per-device set-up: the array's address on the current device, and its contents zeroed once,
// synchronously on `s` before the array is marked ready, so that a first call from any other
// stream (or thread) finds it zero. A set-up cannot synchronise a stream under capture: a first
// call made under graph capture is refused with a message (affx_init does the set-up beforehand).
int noalloc_setup(int dev, hipStream_t s, uint8_t** out) {
  std::lock_guard<std::mutex> lk(g_na_mu);
  if (!g_na_ptr[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    int rc = check_hip(hipStreamIsCapturing(s, &cap), "hipStreamIsCapturing");
    if (rc) return rc;
    if (cap != hipStreamCaptureStatusNone)
      return set_error(AFFX_ERR_ARG, "ffn_decode_noalloc: the scratch array of device %d is not set up; call "
                       "affx_init on that device before capturing", dev);
    void* p = nullptr;
    rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc) return rc;
    if (!p) return set_error(AFFX_ERR_HIP, "ffn_decode_noalloc: no device address for the scratch array");
    hipLaunchKernelGGL(noalloc_zero_kernel, dim3(256), dim3(256), 0, s, (uint4*)p, kNaScratchBytes / 16);
    if ((rc = check_launch("noalloc_zero_kernel"))) return rc;
    if ((rc = check_hip(hipStreamSynchronize(s), "noalloc set-up sync"))) return rc;
    g_na_ptr[dev] = (uint8_t*)p;
  }
  *out = g_na_ptr[dev];
  return AFFX_OK;
}

}  // namespace

namespace affx {

// Called by affx_init for the current device: the set-up happens there, synchronously, so that a
// later call (perhaps under graph capture) finds the array ready.
int noalloc_init_device(int dev) {
  if (dev < 0 || dev >= kNaMaxDev) return AFFX_OK;  // such a device is refused by the entry itself
  uint8_t* p = nullptr;
  return noalloc_setup(dev, nullptr, &p);
}

}  // namespace affx

extern "C" {

int affx_expert_ffn_decode_noalloc(const affx_layer* L, const float* x, uint64_t x_ts, uint64_t x_ds,
                                   uint32_t M, const uint32_t* sel, const float* w, uint32_t K, float* y,
                                   uint64_t y_ts, uint64_t y_ds, int accumulate, void* stream) {
  if (!L) return set_error(AFFX_ERR_ARG, "ffn_decode_noalloc: null layer");
  if (M == 0 || M > kNaMaxTok || K == 0 || (uint64_t)M * K > kNaMaxRoutes || L->hidden > kNaMaxHidden ||
      L->inter > kNaMaxInter)
    return set_error(AFFX_ERR_ARG,
                     "ffn_decode_noalloc: m_tokens %u x top_k %u, hidden %u, inter %u exceed the scratch array "
                     "(m_tokens <= %u, m_tokens * top_k <= %u, hidden <= %u, inter <= %u): use "
                     "affx_expert_ffn_decode with a workspace",
                     M, K, L->hidden, L->inter, kNaMaxTok, kNaMaxRoutes, kNaMaxHidden, kNaMaxInter);
  const size_t need = affx_decode_workspace_size(M, K, L->hidden, L->inter);
  if (need > kNaScratchBytes)
    return set_error(AFFX_ERR_ARG, "ffn_decode_noalloc: needs %zu bytes of scratch, the array holds %llu", need,
                     (unsigned long long)kNaScratchBytes);
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kNaMaxDev) return set_error(AFFX_ERR_ARG, "ffn_decode_noalloc: device id %d", dev);
  uint8_t* ws = nullptr;
  if ((rc = noalloc_setup(dev, (hipStream_t)stream, &ws))) return rc;
  return affx_expert_ffn_decode(L, x, x_ts, x_ds, M, sel, w, K, y, y_ts, y_ds, accumulate, ws,
                                (size_t)kNaScratchBytes, stream);
}

int affx_decode_noalloc_status(int reset, void* stream) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kNaMaxDev) return set_error(AFFX_ERR_ARG, "decode_noalloc_status: device id %d", dev);
  uint8_t* ws = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_na_mu);
    ws = g_na_ptr[dev];
  }
  if (!ws) return AFFX_OK;  // never set up: no call ran on this device
  hipStream_t s = (hipStream_t)stream;
  uint32_t err = 0;
  rc = check_hip(hipMemcpyAsync(&err, ws + kSyncErrWord * 4, 4, hipMemcpyDeviceToHost, s), "noalloc status D2H");
  if (!rc) rc = check_hip(hipStreamSynchronize(s), "noalloc status sync");
  if (rc) return rc;
  if (!err) return AFFX_OK;
  if (reset) {
    // the sync run again as after the set-up (a fill kernel: no memset node if the caller's stream
    // is later captured)
    hipLaunchKernelGGL(noalloc_zero_kernel, dim3(64), dim3(256), 0, s, (uint4*)ws, (uint64_t)(kSyncBytes / 16));
    if ((rc = check_launch("noalloc_zero_kernel"))) return rc;
    if ((rc = check_hip(hipStreamSynchronize(s), "noalloc status sync"))) return rc;
  }
  return set_error(AFFX_ERR_DEVICE, "decode_noalloc_status: an allocation-free decode launch gave up waiting for its "
                   "workgroups (error bits 0x%x); its output was invalid%s", err, reset ? " (state reset)" : "");
}

}  // extern "C"
