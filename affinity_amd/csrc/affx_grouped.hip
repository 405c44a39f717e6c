// Prefill path: the routed experts of a whole chunk, grouped by expert (each expert's weights
// are decoded once per tile of its tokens), on the fp8 MFMA.
//
//   grouped_plan     one workgroup: per-expert counts, exclusive scan, tile lists
//   grouped_place    one workgroup per expert: its (token, route) pairs in token order (stable),
//                    so every slot and every output sum has a fixed order
//   grouped_prep_x   per token: exponent and E4M3 terms of the activation (2 terms are exact for
//                    bf16 input; 3 when a low bf16 term is given)
//   grouped_gateup   (row block of 64 inter rows, token tile): 4 waves x 16 rows of gate and up,
//                    K = hidden in 128-column MFMA steps, 8 token groups per A fragment; epilogue
//                    combines terms, applies row scales, SwiGLU, writes the activation as terms
//   grouped_down     (row block of 64 hidden rows, slot tile): same structure over K = inter,
//                    writes each slot's unweighted down output z[slot]
//   grouped_combine  y[t] (+)= sum_j w[t][j] * z[slot(t, j)] in route order
//
// Reference counterparts: run_batch_device's prefill arm (src/gpu/static_placement.hip:
// 1348-1964): moe_plan_kernel (src/gpu/moe_plan.hip:116-380), batch_quant_fp8_kernel
// (src/gpu/batch_kernels.hip:146-211), expert_gemm_wmma_kernel (src/gpu/expert_kernel.hip:
// 364-825), expert_swiglu_quant_kernel (862-931), expert_scatter_slots_kernel (935-947).
#include "affx_tile.h"

namespace affx {

constexpr int kGroups = 8;         // token groups per tile (one MFMA column block each)
constexpr int kPlanThreads = 1024;

struct Tile {
  uint32_t expert, slot0, n;
};

struct GroupedHdr {
  uint32_t n_slots;
  uint32_t n_tiles1, n_tiles2;
  uint32_t tx;                     // activation terms of the gate/up input (2 or 3)
};

struct GroupedArgs {
  const uint8_t* base;
  uint64_t stride;
  uint64_t off[9];
  uint32_t hidden, inter, n_experts, n_tok, top_k;
  const uint32_t* codebook;
  const GroupedHdr* hdr;
  const uint32_t* offsets;         // [E+1]
  const uint32_t* slot_tok;        // [T*K]
  const int32_t* slot_of;          // [T*K]
  const Tile* tiles1;
  const Tile* tiles2;
  const int32_t* x_sigma;          // [T]
  const uint8_t* xq;               // [T][tx][hidden]
  uint8_t* aq;                     // [slots][3][inter]
  float* z;                        // [slots][hidden]
  const uint8_t* zeros;
  float limit;
  int32_t sigma_a;
  uint32_t tx, tpg1, tpg2;         // terms and tokens per group, gate/up and down
};

// ------------------------------------------------------------------------------------------------
// plan
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kPlanThreads) grouped_plan_kernel(
    const uint32_t* __restrict__ sel, uint32_t n_pairs, uint32_t n_experts, uint32_t tt1,
    uint32_t tt2, uint32_t tx, GroupedHdr* __restrict__ hdr, uint32_t* __restrict__ offsets,
    Tile* __restrict__ tiles1, Tile* __restrict__ tiles2) {
  __shared__ uint32_t cnt[AFFX_MAX_EXPERTS];
  __shared__ uint32_t off[AFFX_MAX_EXPERTS + 1], t1[AFFX_MAX_EXPERTS + 1], t2[AFFX_MAX_EXPERTS + 1];
  const uint32_t tid = threadIdx.x;
  for (uint32_t e = tid; e < AFFX_MAX_EXPERTS; e += kPlanThreads) cnt[e] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < n_pairs; i += kPlanThreads) {
    const uint32_t e = sel[i];
    if (e < n_experts) atomicAdd(&cnt[e], 1u);
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t s = 0, a = 0, b = 0;
    for (uint32_t e = 0; e < n_experts; ++e) {
      off[e] = s; t1[e] = a; t2[e] = b;
      s += cnt[e];
      a += (cnt[e] + tt1 - 1) / tt1;
      b += (cnt[e] + tt2 - 1) / tt2;
    }
    off[n_experts] = s; t1[n_experts] = a; t2[n_experts] = b;
    hdr->n_slots = s;
    hdr->n_tiles1 = a;
    hdr->n_tiles2 = b;
    hdr->tx = tx;
  }
  __syncthreads();
  for (uint32_t e = tid; e <= n_experts; e += kPlanThreads) offsets[e] = off[e];
  for (uint32_t e = tid; e < n_experts; e += kPlanThreads) {
    for (uint32_t k = 0; k < t1[e + 1] - t1[e]; ++k) {
      const uint32_t s0 = off[e] + k * tt1, n = min(tt1, off[e] + cnt[e] - s0);
      tiles1[t1[e] + k] = Tile{e, s0, n};
    }
    for (uint32_t k = 0; k < t2[e + 1] - t2[e]; ++k) {
      const uint32_t s0 = off[e] + k * tt2, n = min(tt2, off[e] + cnt[e] - s0);
      tiles2[t2[e] + k] = Tile{e, s0, n};
    }
  }
}

// One workgroup per expert (plus the padding pass in workgroup n_experts): walks all pairs in
// order and gives this expert's pairs consecutive slots.
__global__ void __launch_bounds__(256) grouped_place_kernel(
    const uint32_t* __restrict__ sel, uint32_t n_pairs, uint32_t top_k, uint32_t n_experts,
    const uint32_t* __restrict__ offsets, uint32_t* __restrict__ slot_tok,
    int32_t* __restrict__ slot_of) {
  const uint32_t e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (e == n_experts) {
    for (uint32_t i = tid; i < n_pairs; i += 256)
      if (sel[i] >= n_experts) slot_of[i] = -1;
    return;
  }
  __shared__ uint32_t wsum[4];
  uint32_t base = offsets[e];
  if (offsets[e + 1] == base) return;
  for (uint32_t c0 = 0; c0 < n_pairs; c0 += 256) {
    const uint32_t i = c0 + tid;
    const bool mine = i < n_pairs && sel[i] == e;
    const uint64_t bal = __ballot(mine);
    const uint32_t before = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wsum[wv] = __popcll(bal);
    __syncthreads();
    uint32_t wofs = 0;
    for (uint32_t q = 0; q < wv; ++q) wofs += wsum[q];
    const uint32_t total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    if (mine) {
      const uint32_t pos = base + wofs + before;
      slot_tok[pos] = i / top_k;
      slot_of[i] = (int32_t)pos;
    }
    base += total;
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------------
// activation terms
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) grouped_prep_x_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ xlo,
                                                             uint32_t hidden, uint32_t tx,
                                                             int32_t* __restrict__ sigma_out,
                                                             uint8_t* __restrict__ xq,
                                                             uint32_t* __restrict__ zeros) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  if (t == 0 && tid < 64) zeros[tid] = 0u;  // the B source of unused columns
  __shared__ float red[4];
  const uint16_t* xr = x + (uint64_t)t * hidden;
  const uint16_t* lr = xlo ? xlo + (uint64_t)t * hidden : nullptr;
  float amax = 0.f;
  for (uint32_t h = tid; h < hidden; h += 256) {
    float v = __uint_as_float((uint32_t)xr[h] << 16);
    if (lr) v += __uint_as_float((uint32_t)lr[h] << 16);
    amax = fmaxf(amax, fabsf(v));
  }
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int sigma = amax > 0.f ? 7 - ilogbf(amax) : 0;
  if (tid == 0) sigma_out[t] = sigma;
  for (uint32_t h4 = tid * 4; h4 < hidden; h4 += 1024) {
    uint32_t q[3] = {0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = __uint_as_float((uint32_t)xr[h4 + i] << 16);
      if (lr) v += __uint_as_float((uint32_t)lr[h4 + i] << 16);
      uint32_t b0, b1, b2;
      split3(ldexpf(v, sigma), b0, b1, b2);
      q[0] |= b0 << (8 * i);
      q[1] |= b1 << (8 * i);
      q[2] |= b2 << (8 * i);
    }
    uint32_t* dst = reinterpret_cast<uint32_t*>(xq + (uint64_t)t * tx * hidden + h4);
    for (uint32_t k = 0; k < tx; ++k) dst[k * (hidden / 4)] = q[k];
  }
}

// ------------------------------------------------------------------------------------------------
// GEMM pieces
// ------------------------------------------------------------------------------------------------

// B source of group g for this lane: column c = token (c / tx) of the group, term c % tx.
__device__ __forceinline__ const u32x4* group_b(const GroupedArgs& A, const uint8_t* src,
                                                uint32_t row_bytes, uint32_t tx, uint32_t tpg,
                                                uint32_t slot0, uint32_t n, uint32_t g,
                                                uint32_t lane, uint64_t col0, bool by_token) {
  const uint32_t c = lane & 15, kg = lane >> 4;
  const uint32_t j = g * tpg + c / tx, tau = c % tx;
  if (c >= tx * tpg || j >= n) return reinterpret_cast<const u32x4*>(A.zeros);
  const uint32_t slot = slot0 + j;
  const uint32_t row = by_token ? A.slot_tok[slot] : slot;
  return reinterpret_cast<const u32x4*>(src + ((uint64_t)row * tx + tau) * row_bytes + col0 +
                                        kg * kSegCols);
}

// Sum of the tx term columns starting at this lane's column (row group of 16 lanes).
__device__ __forceinline__ float combine_cols(float d, uint32_t tx) {
  const float d1 = __shfl_down(d, 1, 16), d2 = __shfl_down(d, 2, 16);
  return tx == 2 ? d + d1 * 0.0625f : d + d1 * 0.0625f + d2 * 0.00390625f;
}

// ------------------------------------------------------------------------------------------------
// gate/up + SwiGLU
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) grouped_gateup_kernel(GroupedArgs A) {
  const uint32_t tile_id = blockIdx.y;
  if (tile_id >= A.hdr->n_tiles1) return;
  const Tile tl = A.tiles1[tile_id];
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t rt = blockIdx.x * 4 + wv;  // 16-row tile of the inter dimension
  const uint32_t nst = A.hidden / kTileCols, tx = A.tx, tpg = A.tpg1;
  const uint32_t ng = (tl.n + tpg - 1) / tpg;
  const uint8_t* ex = A.base + (uint64_t)tl.expert * A.stride;

  __shared__ uint32_t tbl[4 * kLut];
  Unit ug, uu;
  load_unit(ug, ex + A.off[kGateCodes], ex + A.off[kGateFields], (uint64_t)rt * nst, lane);
  load_unit(uu, ex + A.off[kUpCodes], ex + A.off[kUpFields], (uint64_t)rt * nst, lane);
  build_table(tbl, A.codebook);
  __syncthreads();

  v4f acc[2][kGroups];
#pragma unroll
  for (int g = 0; g < kGroups; ++g) acc[0][g] = acc[1][g] = v4f{0.f, 0.f, 0.f, 0.f};

  for (uint32_t S = 0; S < nst; ++S) {
    if (S > 0) {
      load_unit(ug, ex + A.off[kGateCodes], ex + A.off[kGateFields], (uint64_t)rt * nst + S, lane);
      load_unit(uu, ex + A.off[kUpCodes], ex + A.off[kUpFields], (uint64_t)rt * nst + S, lane);
    }
    const u32x4* bp[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g)
      bp[g] = group_b(A, A.xq, A.hidden, tx, tpg, tl.slot0, tl.n, g, lane, (uint64_t)S * kTileCols, true);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      pin(ug);
      pin(uu);
      const v8i ag = decode_step(ug, tbl, m), au = decode_step(uu, tbl, m);
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        if ((uint32_t)g < ng) {
          const v8i b = b_step(bp[g], m);
          acc[0][g] = mfma(ag, b, acc[0][g]);
          acc[1][g] = mfma(au, b, acc[1][g]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // epilogue: lane (col c, row group q) holds rows 16*rt + 4q + v
  const uint32_t c = lane & 15, q = lane >> 4;
  const uint32_t row0 = rt * 16 + 4 * q;
  const uint2 rgv = *reinterpret_cast<const uint2*>(ex + A.off[kGateRs] + (uint64_t)row0 * 2);
  const uint2 ruv = *reinterpret_cast<const uint2*>(ex + A.off[kUpRs] + (uint64_t)row0 * 2);
  const float rg[4] = {__uint_as_float(rgv.x << 16), __uint_as_float(rgv.x & 0xFFFF0000u),
                       __uint_as_float(rgv.y << 16), __uint_as_float(rgv.y & 0xFFFF0000u)};
  const float ru[4] = {__uint_as_float(ruv.x << 16), __uint_as_float(ruv.x & 0xFFFF0000u),
                       __uint_as_float(ruv.y << 16), __uint_as_float(ruv.y & 0xFFFF0000u)};
  const float L = A.limit;
#pragma unroll
  for (int g = 0; g < kGroups; ++g) {
    float sg[4], su[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sg[v] = combine_cols(acc[0][g][v], tx);
      su[v] = combine_cols(acc[1][g][v], tx);
    }
    const uint32_t j = g * tpg + c / tx;
    if ((uint32_t)g < ng && c % tx == 0 && c < tx * tpg && j < tl.n) {
      const uint32_t slot = tl.slot0 + j;
      const int sig = A.x_sigma[A.slot_tok[slot]];
      uint32_t o0 = 0, o1 = 0, o2 = 0;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float gv = ldexpf(sg[v], -sig) * rg[v];
        float uv = ldexpf(su[v], -sig) * ru[v];
        gv = (L < gv) ? L : gv;  // SwiGLU with the asymmetric clamp: src/engine/ops.cpp:47-60
        const float lo = (-L < uv) ? uv : -L;
        uv = (lo < L) ? lo : L;
        const float a = (gv / (1.0f + expf(-gv))) * uv;
        uint32_t b0, b1, b2;
        split3(ldexpf(a, A.sigma_a), b0, b1, b2);
        o0 |= b0 << (8 * v);
        o1 |= b1 << (8 * v);
        o2 |= b2 << (8 * v);
      }
      uint8_t* dst = A.aq + (uint64_t)slot * 3 * A.inter + row0;
      *reinterpret_cast<uint32_t*>(dst) = o0;
      *reinterpret_cast<uint32_t*>(dst + A.inter) = o1;
      *reinterpret_cast<uint32_t*>(dst + 2 * (uint64_t)A.inter) = o2;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// down: z[slot][row] = rs_d[row] * sum_k W_d[row][k] * a[slot][k]
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) grouped_down_kernel(GroupedArgs A) {
  const uint32_t tile_id = blockIdx.y;
  if (tile_id >= A.hdr->n_tiles2) return;
  const Tile tl = A.tiles2[tile_id];
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t rt = blockIdx.x * 4 + wv;  // 16-row tile of the hidden dimension
  const uint32_t nst = A.inter / kTileCols, tpg = A.tpg2;
  const uint32_t ng = (tl.n + tpg - 1) / tpg;
  const uint8_t* ex = A.base + (uint64_t)tl.expert * A.stride;

  __shared__ uint32_t tbl[4 * kLut];
  Unit ud;
  load_unit(ud, ex + A.off[kDownCodes], ex + A.off[kDownFields], (uint64_t)rt * nst, lane);
  build_table(tbl, A.codebook);
  __syncthreads();

  v4f acc[kGroups];
#pragma unroll
  for (int g = 0; g < kGroups; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};
  for (uint32_t S = 0; S < nst; ++S) {
    if (S > 0) load_unit(ud, ex + A.off[kDownCodes], ex + A.off[kDownFields], (uint64_t)rt * nst + S, lane);
    const u32x4* bp[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g)
      bp[g] = group_b(A, A.aq, A.inter, 3, tpg, tl.slot0, tl.n, g, lane, (uint64_t)S * kTileCols, false);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      pin(ud);
      const v8i a = decode_step(ud, tbl, m);
#pragma unroll
      for (int g = 0; g < kGroups; ++g)
        if ((uint32_t)g < ng) acc[g] = mfma(a, b_step(bp[g], m), acc[g]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const uint32_t c = lane & 15, q = lane >> 4;
  const uint32_t row0 = rt * 16 + 4 * q;
  const uint2 rdv = *reinterpret_cast<const uint2*>(ex + A.off[kDownRs] + (uint64_t)row0 * 2);
  const float rd[4] = {__uint_as_float(rdv.x << 16), __uint_as_float(rdv.x & 0xFFFF0000u),
                       __uint_as_float(rdv.y << 16), __uint_as_float(rdv.y & 0xFFFF0000u)};
#pragma unroll
  for (int g = 0; g < kGroups; ++g) {
    float s[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) s[v] = combine_cols(acc[g][v], 3);
    const uint32_t j = g * tpg + c / 3;
    if ((uint32_t)g < ng && c % 3 == 0 && c < 3 * tpg && j < tl.n) {
      float4 o;
      o.x = ldexpf(s[0], -A.sigma_a) * rd[0];
      o.y = ldexpf(s[1], -A.sigma_a) * rd[1];
      o.z = ldexpf(s[2], -A.sigma_a) * rd[2];
      o.w = ldexpf(s[3], -A.sigma_a) * rd[3];
      *reinterpret_cast<float4*>(A.z + (uint64_t)(tl.slot0 + j) * A.hidden + row0) = o;
    }
  }
}

// y[t][h] (+)= sum_j w[t][j] * z[slot(t,j)][h], j ascending.
__global__ void __launch_bounds__(256) grouped_combine_kernel(const float* __restrict__ z,
                                                              const int32_t* __restrict__ slot_of,
                                                              const float* __restrict__ w,
                                                              uint32_t top_k, uint32_t hidden,
                                                              float* __restrict__ y, int accumulate) {
  const uint32_t t = blockIdx.y;
  const uint32_t h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= hidden) return;
  float4 acc = accumulate ? *reinterpret_cast<const float4*>(y + (uint64_t)t * hidden + h)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t j = 0; j < top_k; ++j) {
    const int32_t s = slot_of[t * top_k + j];
    if (s < 0) continue;
    const float wt = w[t * top_k + j];
    const float4 v = *reinterpret_cast<const float4*>(z + (uint64_t)s * hidden + h);
    acc.x += wt * v.x;
    acc.y += wt * v.y;
    acc.z += wt * v.z;
    acc.w += wt * v.w;
  }
  *reinterpret_cast<float4*>(y + (uint64_t)t * hidden + h) = acc;
}

}  // namespace affx

using namespace affx;

namespace {

uint64_t a256(uint64_t v) { return (v + 255) / 256 * 256; }

struct GroupedWs {
  uint64_t hdr, offsets, slot_tok, slot_of, tiles1, tiles2, sigma, zeros, xq, aq, z, total;
  uint32_t max_tiles1, max_tiles2;
};

GroupedWs grouped_ws(uint32_t T, uint32_t K, uint32_t E, uint32_t hidden, uint32_t inter,
                     uint32_t tt1, uint32_t tt2) {
  GroupedWs w;
  const uint64_t P = (uint64_t)T * K;
  w.max_tiles1 = (uint32_t)(P / tt1 + E + 1);
  w.max_tiles2 = (uint32_t)(P / tt2 + E + 1);
  uint64_t o = 0;
  w.hdr = o; o += a256(sizeof(GroupedHdr));
  w.offsets = o; o += a256(4ull * (AFFX_MAX_EXPERTS + 1));
  w.slot_tok = o; o += a256(4 * P);
  w.slot_of = o; o += a256(4 * P);
  w.tiles1 = o; o += a256(sizeof(Tile) * w.max_tiles1);
  w.tiles2 = o; o += a256(sizeof(Tile) * w.max_tiles2);
  w.sigma = o; o += a256(4ull * T);
  w.zeros = o; o += 256;
  w.xq = o; o += a256((uint64_t)T * 3 * hidden);
  w.aq = o; o += a256(P * 3 * inter);
  w.z = o; o += a256(P * 4 * hidden);
  w.total = o;
  return w;
}

// tokens per tile: kGroups column blocks of 16/terms tokens each
uint32_t tpg_of(uint32_t terms) { return 16 / terms; }

}  // namespace

extern "C" {

size_t affx_grouped_workspace_size(uint32_t n_tok, uint32_t top_k, uint32_t n_experts,
                                   uint32_t hidden, uint32_t inter) {
  // sized for the 3-term gate/up input, which needs the most tiles
  return (size_t)grouped_ws(n_tok, top_k, n_experts, hidden, inter, kGroups * tpg_of(3),
                            kGroups * tpg_of(3)).total;
}

int affx_expert_ffn_grouped(const affx_layer* L, const void* x, const void* x_lo, uint32_t T,
                            const uint32_t* sel, const float* w, uint32_t K, float* y,
                            int accumulate, void* ws, size_t ws_bytes, void* stream) {
  if (!L || !x || !sel || !w || !y || !ws || !L->base || !L->codebook)
    return set_error(AFFX_ERR_ARG, "ffn_grouped: null pointer");
  if (T == 0) return AFFX_OK;
  if (K == 0 || K > AFFX_MAX_TOPK || L->n_experts == 0 || L->n_experts > AFFX_MAX_EXPERTS)
    return set_error(AFFX_DECLINED, "ffn_grouped: top_k must be 1..%d and n_experts 1..%d",
                     AFFX_MAX_TOPK, AFFX_MAX_EXPERTS);
  if (L->hidden % kTileCols || L->inter % kTileCols || L->hidden % 64 || L->inter % 64 ||
      L->hidden == 0 || L->inter == 0)
    return set_error(AFFX_DECLINED, "ffn_grouped: hidden and inter must be multiples of 1024");
  if (!(L->swiglu_limit > 0.f) || L->swiglu_limit > 1e6f)
    return set_error(AFFX_DECLINED, "ffn_grouped: needs a SwiGLU clamp limit in (0, 1e6]");
  if ((uint64_t)T * K > (1ull << 31)) return set_error(AFFX_DECLINED, "ffn_grouped: batch too large");
  const uint32_t tx = x_lo ? 3 : 2;
  const uint32_t tt1 = kGroups * tpg_of(tx), tt2 = kGroups * tpg_of(3);
  const GroupedWs lay = grouped_ws(T, K, L->n_experts, L->hidden, L->inter, tt1, tt2);
  if (ws_bytes < lay.total)
    return set_error(AFFX_ERR_ARG, "ffn_grouped: workspace %zu < %llu bytes", ws_bytes,
                     (unsigned long long)lay.total);
  uint64_t off9[9];
  const uint64_t stride = affx_expert_layout(L->hidden, L->inter, off9, nullptr);
  if (L->stride < stride) return set_error(AFFX_ERR_ARG, "ffn_grouped: layer stride below expert size");

  uint8_t* b = (uint8_t*)ws;
  hipStream_t s = (hipStream_t)stream;
  GroupedArgs A;
  A.base = (const uint8_t*)L->base;
  A.stride = L->stride;
  for (int i = 0; i < 9; ++i) A.off[i] = off9[i];
  A.hidden = L->hidden;
  A.inter = L->inter;
  A.n_experts = L->n_experts;
  A.n_tok = T;
  A.top_k = K;
  A.codebook = (const uint32_t*)L->codebook;
  A.hdr = (const GroupedHdr*)(b + lay.hdr);
  A.offsets = (const uint32_t*)(b + lay.offsets);
  A.slot_tok = (const uint32_t*)(b + lay.slot_tok);
  A.slot_of = (const int32_t*)(b + lay.slot_of);
  A.tiles1 = (const Tile*)(b + lay.tiles1);
  A.tiles2 = (const Tile*)(b + lay.tiles2);
  A.x_sigma = (const int32_t*)(b + lay.sigma);
  A.xq = b + lay.xq;
  A.aq = b + lay.aq;
  A.z = (float*)(b + lay.z);
  A.zeros = b + lay.zeros;
  A.limit = L->swiglu_limit;
  A.sigma_a = 7 - ilogbf(L->swiglu_limit * L->swiglu_limit);
  A.tx = tx;
  A.tpg1 = tpg_of(tx);
  A.tpg2 = tpg_of(3);

  const uint32_t P = T * K;
  hipLaunchKernelGGL(grouped_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, sel, P, L->n_experts,
                     tt1, tt2, tx, (GroupedHdr*)(b + lay.hdr), (uint32_t*)(b + lay.offsets),
                     (Tile*)(b + lay.tiles1), (Tile*)(b + lay.tiles2));
  int rc = check_launch("grouped_plan_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(grouped_place_kernel, dim3(L->n_experts + 1), dim3(256), 0, s, sel, P, K,
                     L->n_experts, (const uint32_t*)(b + lay.offsets), (uint32_t*)(b + lay.slot_tok),
                     (int32_t*)(b + lay.slot_of));
  if ((rc = check_launch("grouped_place_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_prep_x_kernel, dim3(T), dim3(256), 0, s, (const uint16_t*)x,
                     (const uint16_t*)x_lo, L->hidden, tx, (int32_t*)(b + lay.sigma), b + lay.xq,
                     (uint32_t*)(b + lay.zeros));
  if ((rc = check_launch("grouped_prep_x_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_gateup_kernel, dim3(L->inter / 64, lay.max_tiles1), dim3(256), 0, s, A);
  if ((rc = check_launch("grouped_gateup_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_down_kernel, dim3(L->hidden / 64, lay.max_tiles2), dim3(256), 0, s, A);
  if ((rc = check_launch("grouped_down_kernel"))) return rc;
  hipLaunchKernelGGL(grouped_combine_kernel, dim3((L->hidden / 4 + 255) / 256, T), dim3(256), 0, s,
                     (const float*)(b + lay.z), (const int32_t*)(b + lay.slot_of), w, K, L->hidden,
                     y, accumulate);
  return check_launch("grouped_combine_kernel");
}

}  // extern "C"
