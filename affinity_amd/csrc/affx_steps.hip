// The reference's separable steps of its batched expert pipeline, as standalone entries for a
// caller that drives that pipeline step by step (its run_batch_device does: gather -> W8A8 gate/up
// GEMM -> SwiGLU + requantise -> W8A8 down GEMM -> fixed-order scatter,
// src/gpu/static_placement.hip:1856-1914). The library's own prefill fuses these into its grouped
// GEMM and combine; these entries keep the reference's formats and results:
//   affx_expert_swiglu_quant   expert_swiglu_quant_hip   (src/gpu/expert_kernel_hip.h:238-240)
//   affx_expert_scatter_slots  expert_scatter_slots_hip  (src/gpu/expert_kernel_hip.h:249-251)
//   affx_expert_gather_tokens  expert_gather_tokens_hip  (src/gpu/expert_kernel_hip.h:255-256)
// All three are bandwidth-bound passes over their arrays.
#include "affx_common.h"

namespace affx {

__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// SwiGLU x router weight over a dim-major [dim][total] pair of bf16 arenas, then one E4M3
// requantisation per (slot, 128-row band): scale = max |v| / 448 (1 when the band is zero), bytes
// = E4M3(clamp(v / scale, +-448)) slot-major [total][dim]. A workgroup takes 64 slots of one band:
// wave q reads rows 32 q .. 32 q + 31 of the band (64 consecutive slots per row, one 128-byte
// read), keeps the values in LDS and its per-slot maxima; then each thread writes 16 bytes of one
// slot's band (the 128 bytes of a slot are one run). The float operations and their order are the
// reference's (expert_kernel.hip:862-931), so the bytes agree with its CPU restatement up to expf.
constexpr uint32_t kSqSlots = 64;

__global__ void __launch_bounds__(256) swiglu_quant_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                           const float* __restrict__ w, uint8_t* __restrict__ out,
                                                           float* __restrict__ scales, uint32_t dim, uint32_t total,
                                                           float limit) {
  __shared__ float tile[128][kSqSlots + 1];
  __shared__ float pmax[4][kSqSlots];
  __shared__ float sinv[kSqSlots];
  const uint32_t tid = threadIdx.x, s = tid & 63u, q = tid >> 6;
  const uint32_t s0 = blockIdx.x * kSqSlots, sl = s0 + s, kb = blockIdx.y, nkb = dim / 128u;
  const bool ok = sl < total;
  const float wv = (ok && w) ? w[sl] : 1.0f;
  float m = 0.0f;
  for (uint32_t i = 0; i < 32u; ++i) {
    const uint32_t k = 32u * q + i;
    float v = 0.0f;
    if (ok) {
      const uint64_t o = (uint64_t)(kb * 128u + k) * total + sl;
      float gv = bf16f(g[o]), uv = bf16f(u[o]);
      if (limit > 0.0f) {
        gv = fminf(gv, limit);
        uv = fminf(limit, fmaxf(-limit, uv));
      }
      v = (gv / (1.0f + expf(-gv))) * uv * wv;
    }
    tile[k][s] = v;
    m = fmaxf(m, fabsf(v));
  }
  pmax[q][s] = m;
  __syncthreads();
  if (tid < kSqSlots) {
    const float mm = fmaxf(fmaxf(pmax[0][tid], pmax[1][tid]), fmaxf(pmax[2][tid], pmax[3][tid]));
    const float sc = mm > 0.0f ? mm * (1.0f / 448.0f) : 1.0f;
    if (s0 + tid < total) scales[(uint64_t)(s0 + tid) * nkb + kb] = sc;
    sinv[tid] = 1.0f / sc;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t cidx = tid + 256u * (uint32_t)j, ss = cidx >> 3, p = cidx & 7u;
    if (s0 + ss < total) {
      const float inv = sinv[ss];
      uint32_t wo[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = fminf(fmaxf(tile[16u * p + 4u * h + e][ss] * inv, -448.0f), 448.0f);
        int pk = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
        pk = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], pk, true);
        wo[h] = (uint32_t)pk;
      }
      *reinterpret_cast<uint4*>(out + (uint64_t)(s0 + ss) * dim + kb * 128u + 16u * p) = uint4{wo[0], wo[1], wo[2], wo[3]};
    }
  }
}

// block[h][t] += the sum, in ord order from zero, of the bf16 slot outputs y[h][ord[i]] for
// i in run[t] .. run[t+1]-1 (tokens without slots untouched). One workgroup per (row h, 256
// tokens); a row's slots are one contiguous run, so its scattered reads stay in the caches.
__global__ void __launch_bounds__(256) scatter_slots_kernel(const uint16_t* __restrict__ y, float* __restrict__ block,
                                                            const uint32_t* __restrict__ ord,
                                                            const uint32_t* __restrict__ run, uint32_t nb_tok,
                                                            uint32_t nb_stride, uint32_t total) {
  const uint32_t h = blockIdx.y, t = blockIdx.x * 256u + threadIdx.x;
  if (t >= nb_tok) return;
  const uint32_t a = run[t], b = run[t + 1];
  if (a == b) return;
  const uint16_t* __restrict__ row = y + (uint64_t)h * total;
  float acc = 0.0f;
  for (uint32_t i = a; i < b; ++i) acc += bf16f(row[ord[i]]);
  block[(uint64_t)h * nb_stride + t] += acc;
}

// dst[c][t] = src[c][tok[t]]: nt token columns of a dim-major [dim][nb] arena into a compact
// [dim][nt] tile; a thread per element, consecutive threads consecutive tokens of one row.
__global__ void __launch_bounds__(256) gather_tokens_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                            const uint32_t* __restrict__ tok, uint32_t dim,
                                                            uint32_t nb, uint32_t nt) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= (uint64_t)dim * nt) return;
  const uint32_t c = (uint32_t)(i / nt), t = (uint32_t)(i % nt);
  dst[i] = src[(uint64_t)c * nb + tok[t]];
}

}  // namespace affx

using namespace affx;

extern "C" {

int affx_expert_swiglu_quant(const uint16_t* g, const uint16_t* u, const float* w, uint8_t* out, float* scales,
                             uint32_t dim, uint32_t total, float limit, void* stream) {
  if (!dim || !total) return AFFX_OK;
  if (!g || !u || !out || !scales) return set_error(AFFX_ERR_ARG, "swiglu_quant: null pointer");
  if (dim % 128u) return set_error(AFFX_ERR_ARG, "swiglu_quant: dim %u is not a multiple of 128", dim);
  if ((reinterpret_cast<uintptr_t>(out) & 15u) != 0) return set_error(AFFX_ERR_ARG, "swiglu_quant: out must be 16-byte aligned");
  hipLaunchKernelGGL(swiglu_quant_kernel, dim3((total + kSqSlots - 1) / kSqSlots, dim / 128u), dim3(256), 0,
                     (hipStream_t)stream, g, u, w, out, scales, dim, total, limit);
  return check_launch("swiglu_quant_kernel");
}

int affx_expert_scatter_slots(const uint16_t* y, float* block, const uint32_t* ord, const uint32_t* run,
                              uint32_t dim, uint32_t nb_tok, uint32_t nb_stride, uint32_t total, void* stream) {
  if (!dim || !nb_tok || !total) return AFFX_OK;
  if (!y || !block || !ord || !run) return set_error(AFFX_ERR_ARG, "scatter_slots: null pointer");
  if (nb_stride < nb_tok) return set_error(AFFX_ERR_ARG, "scatter_slots: nb_stride %u < nb_tok %u", nb_stride, nb_tok);
  if (dim > 65535u) return set_error(AFFX_ERR_ARG, "scatter_slots: dim %u above 65535", dim);
  hipLaunchKernelGGL(scatter_slots_kernel, dim3((nb_tok + 255u) / 256u, dim), dim3(256), 0, (hipStream_t)stream, y,
                     block, ord, run, nb_tok, nb_stride, total);
  return check_launch("scatter_slots_kernel");
}

int affx_expert_gather_tokens(const float* src, float* dst, const uint32_t* tok, uint32_t dim, uint32_t nb,
                              uint32_t nt, void* stream) {
  if (!nt || !dim) return AFFX_OK;
  if (!src || !dst || !tok) return set_error(AFFX_ERR_ARG, "gather_tokens: null pointer");
  const uint64_t n = (uint64_t)dim * nt;
  hipLaunchKernelGGL(gather_tokens_kernel, dim3((uint32_t)((n + 255u) / 256u)), dim3(256), 0, (hipStream_t)stream, src,
                     dst, tok, dim, nb, nt);
  return check_launch("gather_tokens_kernel");
}

}  // extern "C"
