// Routing on the device: the router's top-k over a batch's logits, one wave per token, writing
// the [n_tok][top_k] expert ids and weights that the decode and grouped entries read, so a layer
// goes from logits to expert output without routes passing through the host.
//
// Two rules:
//  * the engine's (src/engine/ops.cpp:62-92, the device form src/gpu/batch_kernels.hip:2964-3031):
//    score = sqrt(softplus(logit)) with the x > 20 guard; the k best of score + bias (the bias
//    chooses, it never weighs), ties to the lower id; weight = score * inv * routed_scaling with
//    inv = 1 / (sum of the k scores, in double, floored at the fp16 least normal) when the
//    weights are renormalised, else 1;
//  * the benchmark configs' softmax top-k: the k largest logits (ties to the lower id), weights
//    the softmax over those k, in double.
#include "affx_common.h"

namespace affx {

constexpr int kRouteWaves = 4;                           // tokens per 256-thread workgroup
constexpr int kRouteNV = AFFX_MAX_EXPERTS / 64;          // experts per lane (8)

// (key, id) a better than (key, id) b: key descending, then id ascending; id ~0u is "none".
__device__ __forceinline__ bool route_better(float ka, uint32_t ia, float kb, uint32_t ib) {
  if (ib == ~0u) return ia != ~0u;
  if (ia == ~0u) return false;
  if (ka != kb) return ka > kb;
  return ia < ib;
}

// The engine router's score. expf and log1pf are evaluated in double and rounded once, which is
// within an ulp of the host's float functions (their results are not always correctly rounded).
__device__ __forceinline__ float route_score(float x) {
  if (x > 20.0f) return sqrtf(x);
  const float e = (float)exp((double)x);
  const float sp = (float)log1p((double)e);
  return sqrtf(sp);
}

template <int RULE>
__global__ void __launch_bounds__(kRouteWaves * 64) route_topk_kernel(
    const float* __restrict__ logits, uint64_t tok_stride, uint64_t exp_stride, const float* __restrict__ bias,
    uint32_t n_tok, uint32_t n_expert, uint32_t k, int norm_topk_prob, float routed_scaling,
    uint32_t* __restrict__ sel, float* __restrict__ wout) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * kRouteWaves + (threadIdx.x >> 6);
  if (t >= n_tok) return;  // (whole waves)
  // lane holds experts e = lane + 64 v
  float key[kRouteNV], val[kRouteNV];
#pragma unroll
  for (int v = 0; v < kRouteNV; ++v) {
    const uint32_t e = lane + 64u * v;
    const bool in = e < n_expert;
    const float x = in ? logits[(uint64_t)t * tok_stride + (uint64_t)e * exp_stride] : 0.0f;
    if constexpr (RULE == AFFX_ROUTE_ENGINE) {
      val[v] = in ? route_score(x) : 0.0f;
      key[v] = val[v] + (bias && in ? bias[e] : 0.0f);
    } else {
      val[v] = x;
      key[v] = x;
    }
  }
  uint32_t taken = 0;  // bit v: expert lane + 64 v already chosen
  uint32_t ids[AFFX_MAX_TOPK];
  float vals[AFFX_MAX_TOPK];
  for (uint32_t r = 0; r < k; ++r) {
    float bk = 0.0f, bv = 0.0f;
    uint32_t bi = ~0u;
#pragma unroll
    for (int v = 0; v < kRouteNV; ++v) {
      const uint32_t e = lane + 64u * v;
      if (e < n_expert && !((taken >> v) & 1u) && route_better(key[v], e, bk, bi)) {
        bk = key[v];
        bi = e;
        bv = val[v];
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ok = __shfl_xor(bk, o), ov = __shfl_xor(bv, o);
      const uint32_t oi = __shfl_xor(bi, o);
      if (route_better(ok, oi, bk, bi)) { bk = ok; bi = oi; bv = ov; }
    }
    // every lane holds the same winner now
    if (bi == ~0u) break;
    if ((bi & 63u) == lane) taken |= 1u << (bi >> 6);
    ids[r] = bi;
    vals[r] = bv;
  }
  if (lane == 0) {
    if constexpr (RULE == AFFX_ROUTE_ENGINE) {
      double sum = 0.0;
      for (uint32_t j = 0; j < k; ++j) sum += vals[j];
      if (sum < 6.103515625e-5) sum = 6.103515625e-5;
      const double inv = norm_topk_prob ? 1.0 / sum : 1.0;
      for (uint32_t j = 0; j < k; ++j) {
        sel[(uint64_t)t * k + j] = ids[j];
        wout[(uint64_t)t * k + j] = (float)((double)vals[j] * inv * (double)routed_scaling);
      }
    } else {
      // softmax over the k: the first is the largest logit of all
      double ex[AFFX_MAX_TOPK], sum = 0.0;
      for (uint32_t j = 0; j < k; ++j) {
        ex[j] = exp((double)vals[j] - (double)vals[0]);
        sum += ex[j];
      }
      for (uint32_t j = 0; j < k; ++j) {
        sel[(uint64_t)t * k + j] = ids[j];
        wout[(uint64_t)t * k + j] = (float)(ex[j] / sum);
      }
    }
  }
}

}  // namespace affx

using namespace affx;

extern "C" int affx_route_topk(const float* logits, uint64_t tok_stride, uint64_t expert_stride,
                               const float* bias, uint32_t n_tok, uint32_t n_expert, uint32_t top_k, int rule,
                               int norm_topk_prob, float routed_scaling, uint32_t* sel, float* w,
                               void* stream) {
  if (!logits || !sel || !w) return set_error(AFFX_ERR_ARG, "route_topk: null pointer");
  if (n_tok == 0) return AFFX_OK;
  if (n_expert == 0 || n_expert > AFFX_MAX_EXPERTS || top_k == 0 || top_k > AFFX_MAX_TOPK || top_k > n_expert)
    return set_error(AFFX_DECLINED, "route_topk: n_expert must be 1..%d and top_k 1..min(%d, n_expert)",
                     AFFX_MAX_EXPERTS, AFFX_MAX_TOPK);
  if (rule != AFFX_ROUTE_ENGINE && rule != AFFX_ROUTE_SOFTMAX)
    return set_error(AFFX_ERR_ARG, "route_topk: unknown rule %d", rule);
  const dim3 grid((n_tok + kRouteWaves - 1) / kRouteWaves), blk(kRouteWaves * 64);
  hipStream_t s = (hipStream_t)stream;
  if (rule == AFFX_ROUTE_ENGINE)
    hipLaunchKernelGGL(route_topk_kernel<AFFX_ROUTE_ENGINE>, grid, blk, 0, s, logits, tok_stride, expert_stride,
                       bias, n_tok, n_expert, top_k, norm_topk_prob, routed_scaling, sel, w);
  else
    hipLaunchKernelGGL(route_topk_kernel<AFFX_ROUTE_SOFTMAX>, grid, blk, 0, s, logits, tok_stride, expert_stride,
                       bias, n_tok, n_expert, top_k, norm_topk_prob, routed_scaling, sel, w);
  return check_launch("route_topk_kernel");
}
