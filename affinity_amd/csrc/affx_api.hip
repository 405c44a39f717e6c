// The engine hook: an ExpertFfnBatch-shaped entry (src/engine/model.h:664-666) over the decode
// and grouped paths, reading and accumulating the engine's dim-major f32 arenas.
#include "affx_common.h"

namespace affx {

// d_x f32 [hidden][nb_stride] (dim-major) -> bf16 hi and lo token-major [n][hidden]:
// hi = bf16_RNE(x), lo = bf16_RNE(x - hi), so hi + lo carries 16 significant bits of x.
__global__ void __launch_bounds__(256) split_bf16_kernel(const float* __restrict__ x,
                                                         uint32_t nb_stride, uint32_t n,
                                                         uint32_t hidden, uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)n * hidden) return;
  const uint32_t t = (uint32_t)(i / hidden), h = (uint32_t)(i % hidden);
  const float v = x[(uint64_t)h * nb_stride + t];
  const uint32_t u = __float_as_uint(v);
  const uint16_t a = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  const float r = v - __uint_as_float((uint32_t)a << 16);
  const uint32_t ur = __float_as_uint(r);
  hi[i] = a;
  lo[i] = (uint16_t)((ur + 0x7FFFu + ((ur >> 16) & 1u)) >> 16);
}

// d_block[h][t] += y[t][h]
__global__ void __launch_bounds__(256) add_transposed_kernel(const float* __restrict__ y, uint32_t n,
                                                             uint32_t hidden, float* __restrict__ block,
                                                             uint32_t nb_stride) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)n * hidden) return;
  const uint32_t h = (uint32_t)(i / n), t = (uint32_t)(i % n);
  block[(uint64_t)h * nb_stride + t] += y[(uint64_t)t * hidden + h];
}

}  // namespace affx

using namespace affx;

extern "C" {

// Hook workspace. Decode: [decode workspace][routes][weights]; the decode workspace starts at
// offset 0, so its sync run (counter and release flags, which persist between calls and must stay
// zero) is at the same bytes in every call whatever the batch. Prefill: [sync run, untouched]
// [routes][weights][x hi][x lo][y][grouped workspace], so a prefill call never writes those bytes.
namespace {
struct HookWs {
  uint64_t sel, w, hi, lo, y, inner, need;
};
HookWs hook_ws(uint32_t nb, uint32_t k, uint32_t n_experts, uint32_t hidden, uint32_t inter) {
  HookWs h{};
  const uint64_t pairs = (uint64_t)nb * k;
  if (nb <= AFFX_MAX_DECODE_TOKENS) {
    h.inner = 0;
    h.sel = a256(affx_decode_workspace_size(nb, k, hidden, inter));
    h.w = h.sel + a256(4 * pairs);
    h.need = h.w + a256(4 * pairs);
  } else {
    h.sel = a256(kSyncBytes);
    h.w = h.sel + a256(4 * pairs);
    h.hi = h.w + a256(4 * pairs);
    h.lo = h.hi + a256(2ull * nb * hidden);
    h.y = h.lo + a256(2ull * nb * hidden);
    h.inner = h.y + a256(4ull * nb * hidden);
    h.need = h.inner + affx_grouped_workspace_size(nb, k, n_experts, hidden, inter);
  }
  return h;
}
}  // namespace

size_t affx_batch_workspace_size(uint32_t nb, uint32_t k, uint32_t n_experts, uint32_t hidden,
                                 uint32_t inter) {
  return (size_t)hook_ws(nb, k, n_experts, hidden, inter).need;
}

uint32_t affx_expert_ffn_batch(void* ctx_, uint32_t layer, const uint32_t* sel, const float* w,
                               uint32_t nb, uint32_t k, uint8_t* handled) {
  const affx_engine_ctx* ctx = (const affx_engine_ctx*)ctx_;
  if (!ctx || !sel || !w || !handled || !ctx->layers || !ctx->d_x || !ctx->d_block || !ctx->workspace) {
    set_error(AFFX_ERR_ARG, "ffn_batch: null pointer");
    return 0;
  }
  if (layer >= ctx->n_layers || nb == 0 || k == 0 || k > AFFX_MAX_TOPK || nb > ctx->nb_stride) {
    set_error(AFFX_ERR_ARG, "ffn_batch: layer %u / batch %u x %u out of range", layer, nb, k);
    return 0;
  }
  const affx_layer* L = &ctx->layers[layer];
  hipStream_t s = (hipStream_t)ctx->stream;
  uint8_t* ws = (uint8_t*)ctx->workspace;
  const uint64_t pairs = (uint64_t)nb * k;
  const bool decode = nb <= AFFX_MAX_DECODE_TOKENS;
  const HookWs h = hook_ws(nb, k, L->n_experts, L->hidden, L->inter);
  const uint64_t o_sel = h.sel, o_w = h.w, o_hi = h.hi, o_lo = h.lo, o_y = h.y, o_inner = h.inner;
  if (ctx->workspace_bytes < h.need) {
    set_error(AFFX_ERR_ARG, "ffn_batch: workspace %zu < %llu bytes", ctx->workspace_bytes,
              (unsigned long long)h.need);
    return 0;
  }
  if (check_hip(hipMemcpyAsync(ws + o_sel, sel, 4 * pairs, hipMemcpyHostToDevice, s), "routes H2D") ||
      check_hip(hipMemcpyAsync(ws + o_w, w, 4 * pairs, hipMemcpyHostToDevice, s), "weights H2D"))
    return 0;
  int rc;
  if (decode) {
    rc = affx_expert_ffn_decode(L, ctx->d_x, 1, ctx->nb_stride, nb, (const uint32_t*)(ws + o_sel),
                                (const float*)(ws + o_w), k, ctx->d_block, 1, ctx->nb_stride, 1,
                                ws + o_inner, o_sel, s);
  } else {
    const uint64_t tot = (uint64_t)nb * L->hidden;
    hipLaunchKernelGGL(split_bf16_kernel, dim3((uint32_t)((tot + 255) / 256)), dim3(256), 0, s, ctx->d_x,
                       ctx->nb_stride, nb, L->hidden, (uint16_t*)(ws + o_hi), (uint16_t*)(ws + o_lo));
    if ((rc = check_launch("split_bf16_kernel"))) return 0;
    rc = affx_expert_ffn_grouped(L, ws + o_hi, ws + o_lo, nb, (const uint32_t*)(ws + o_sel),
                                 (const float*)(ws + o_w), k, (float*)(ws + o_y), 0, ws + o_inner,
                                 ctx->workspace_bytes - o_inner, s);
    if (rc == AFFX_OK) {
      hipLaunchKernelGGL(add_transposed_kernel, dim3((uint32_t)((tot + 255) / 256)), dim3(256), 0, s,
                         (const float*)(ws + o_y), nb, L->hidden, ctx->d_block, ctx->nb_stride);
      rc = check_launch("add_transposed_kernel");
    }
  }
  if (rc != AFFX_OK) return 0;
  // the decode's error word comes back with the sync the hook does anyway (routes are host
  // memory, so the engine waits for the layer regardless): a wait that gave up fails the call
  uint32_t err = 0;
  if (decode && check_hip(hipMemcpyAsync(&err, ws + kSyncErrWord * 4, 4, hipMemcpyDeviceToHost, s), "status D2H"))
    return 0;
  if (check_hip(hipStreamSynchronize(s), "ffn_batch sync")) return 0;
  if (err) {
    decode_sync_reset(ws, s);
    set_error(AFFX_ERR_DEVICE, "ffn_batch: layer %u: the decode's workgroups gave up waiting for each "
              "other (error bits 0x%x; the device did not hold the grid resident); output invalid", layer, err);
    return 0;
  }
  uint32_t taken = 0;
  for (uint64_t i = 0; i < pairs; ++i)
    if (sel[i] < L->n_experts) {
      handled[i] = 1;
      ++taken;
    }
  return taken;
}

int affx_decode_status(void* workspace, int reset, void* stream) {
  if (!workspace) return set_error(AFFX_ERR_ARG, "decode_status: null workspace");
  hipStream_t s = (hipStream_t)stream;
  uint32_t err = 0;
  int rc = check_hip(hipMemcpyAsync(&err, (uint8_t*)workspace + kSyncErrWord * 4, 4, hipMemcpyDeviceToHost, s),
                     "decode_status D2H");
  if (!rc) rc = check_hip(hipStreamSynchronize(s), "decode_status sync");
  if (rc) return rc;
  if (!err) return AFFX_OK;
  if (reset && (rc = decode_sync_reset(workspace, s))) return rc;
  if (reset && (rc = check_hip(hipStreamSynchronize(s), "decode_status sync"))) return rc;
  return set_error(AFFX_ERR_DEVICE, "decode_status: a decode launch gave up waiting for its workgroups "
                   "(error bits 0x%x); its output was invalid%s", err, reset ? " (state reset)" : "");
}

}  // extern "C"
