// Decode path (M <= 8 tokens, top-k routing): fused unpack -> codebook dequant -> fp8 MFMA for
// gate/up -> SwiGLU -> down -> weighted combine. Three kernels, stream-ordered:
//
//   decode_prep    plan (distinct experts by first occurrence, token masks, summed weights) and every
//                  token's activation split into three exact-ish E4M3 terms (xq)
//   decode_gateup  grid (row tile of inter, expert slot); 4 waves = 4 column super-segments;
//                  gate and up tiles decoded from the packed codes through an LDS codebook and
//                  multiplied on the fp8 MFMA; fixed-order cross-wave sum, row scale, SwiGLU;
//                  the activation is written back as E4M3 terms (aq)
//   decode_down    grid (row tile of hidden); waves stride over (slot, super-segment) units,
//                  combine terms * row scale * route weight per token, fixed-order cross-wave sum
//
// Why fp8 MFMA at batch 1: a decoded weight is a codebook E4M3 byte with +s added to its
// exponent and the sign flipped, i.e. still an exact E4M3 value, so the weight side needs no
// conversion at all. The activation side is carried as t0 + t1/16 + t2/256 in three B columns
// (five tokens per 16-column MFMA), which keeps the product error near 2^-12 relative while the
// VALU only does code extraction, one LDS lookup and one xor-add per four weights.
//
// Reference counterparts: expert_ffn_hip (src/gpu/expert_kernel.hip:2737-2808) with its
// tr_mat_dot_rb GEMV (1084-1188), swiglu_all_kernel (114-129) and expert_gemv_kernel_tr
// (1201-1258); the fixed-order reductions follow the reference's no-atomics rule (1219-1244).
#include "affx_tile.h"

namespace affx {

// Experts of the pointer-table form (the reference's DeviceExpert arrays): at most this many.
constexpr uint32_t kTblMax = 16;

struct DecodeArgs {
  const uint8_t* base;  // layer expert pool, device layout
  uint64_t stride;
  uint64_t off[9];      // plane offsets inside an expert
  // Pointer-table form: n_tbl > 0 means expert e's plane p is at tbl[e][p] (any device addresses,
  // each plane in device layout) instead of base + e * stride + off[p].
  uint32_t n_tbl;
  const uint8_t* tbl[kTblMax][9];
  uint32_t hidden, inter, m_tokens;
  const uint32_t* codebook;
  const DecodePlan* plan;
  const uint8_t* xq;    // [M][3][hidden]
  const float* x;       // one token's activation (the pointer-table form: its gate/up makes the terms)
  uint8_t* aq;          // [slot][M][3][inter]
  const uint8_t* zeros; // 256 zero bytes: the B source of unused columns
  float limit;
  int32_t sigma_a;      // exponent applied to the SwiGLU output before its E4M3 split
  float* y;
  uint64_t y_ts, y_ds;
  int accumulate;
};

// Plane p of expert e (e uniform across the wave: a scalar load from the kernel arguments in the
// pointer-table form).
__device__ __forceinline__ const uint8_t* plane_ptr(const DecodeArgs& A, uint32_t e, int p) {
  return A.n_tbl ? A.tbl[e < kTblMax ? e : 0][p] : A.base + (uint64_t)e * A.stride + A.off[p];
}

// ------------------------------------------------------------------------------------------------
// prep: blocks 0 .. M*nst-1 split one (token, 1024-column super-segment) of the activation into
// three E4M3 terms with their own exponent; the last block builds the plan.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) decode_prep_kernel(const float* __restrict__ x, uint64_t xts,
                                                          uint64_t xds, uint32_t M,
                                                          const uint32_t* __restrict__ sel,
                                                          const float* __restrict__ w, uint32_t K,
                                                          uint32_t n_experts, uint32_t hidden,
                                                          DecodePlan* __restrict__ plan,
                                                          uint8_t* __restrict__ xq,
                                                          uint8_t* __restrict__ zeros) {
  const uint32_t nst = hidden / kTileCols, tid = threadIdx.x;
  if (blockIdx.x < M * nst) {
    const uint32_t t = blockIdx.x / nst, S = blockIdx.x % nst;
    __shared__ float red[4];
    const int sigma = segment_terms(x, xts, xds, t, S, hidden, xq, red);
    if (tid == 0) plan->x_sigma[t][S] = sigma;
    return;
  }

  // ---- the plan: the distinct experts of the batch in order of first occurrence in the route
  // list (the persistent decode kernel uses the same order, so both give identical sums) ---------
  __shared__ uint32_t sel_l[kMaxSlots];
  __shared__ uint32_t first_l[kMaxSlots];
  __shared__ uint32_t first_slot[kMaxSlots];  // slot of a first-occurrence route
  __shared__ uint32_t rank_l[kMaxSlots];      // slot of every route
  __shared__ uint32_t slot_expert[kMaxSlots];
  __shared__ uint32_t ns_l;
  if (tid < 64) reinterpret_cast<uint32_t*>(zeros)[tid] = 0u;  // the B source of unused columns
  const uint32_t R = M * K;
  if (tid < R) {
    const uint32_t e = sel ? sel[tid] : tid;  // no route list: route j names expert j
    sel_l[tid] = e < n_experts ? e : ~0u;
  }
  __syncthreads();
  if (tid < R) {
    const uint32_t e = sel_l[tid];
    bool dup = false;
    for (uint32_t j = 0; j < tid; ++j) dup = dup || sel_l[j] == e;
    first_l[tid] = e != ~0u && !dup;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t ns = 0;
    for (uint32_t r = 0; r < R; ++r)
      if (first_l[r]) { first_slot[r] = ns; slot_expert[ns] = sel_l[r]; ++ns; }
    ns_l = ns;
    plan->n_slots = ns;
    plan->m_tokens = M;
  }
  __syncthreads();
  if (tid < R) {
    // a repeated expert takes the slot of its first occurrence
    const uint32_t e = sel_l[tid];
    uint32_t s = ~0u;
    for (uint32_t j = 0; j <= tid && e != ~0u; ++j)
      if (first_l[j] && sel_l[j] == e) s = first_slot[j];
    rank_l[tid] = s;
  }
  __syncthreads();
  // one thread per slot: which tokens it serves, with the summed weight of every route to it
  // (a repeated expert counts once per route, summed in route order)
  const uint32_t ns = ns_l;
  if (tid < ns) {
    plan->expert[tid] = slot_expert[tid];
    uint32_t mask = 0;
    for (uint32_t t = 0; t < kMaxTok; ++t) {
      float ws = 0.f;
      if (t < M)
        for (uint32_t j = 0; j < K; ++j)
          if (rank_l[t * K + j] == tid) { ws += w[t * K + j]; mask |= 1u << t; }
      plan->w[tid][t] = ws;
    }
    plan->tok_mask[tid] = mask;
  }
}

// ------------------------------------------------------------------------------------------------
// shared pieces of the two GEMV kernels are in affx_tile.h
// ------------------------------------------------------------------------------------------------

// y = x - low terms: the value of three E4M3 terms t0 + t1/16 + t2/256 from a lane's column c
// and its two right neighbours (same 16-lane row group).
__device__ __forceinline__ float combine_terms(float d) {
  const float d1 = row_shl<1>(d), d2 = row_shl<2>(d);  // (DPP row shifts)
  return d + d1 * 0.0625f + d2 * 0.00390625f;
}

// ------------------------------------------------------------------------------------------------
// gate/up + SwiGLU
// ------------------------------------------------------------------------------------------------
// XL (the pointer-table form, one token): the activation terms are made by every workgroup in its
// own LDS from x, with the prep kernel's split (the same bits), instead of read from the caller's
// scratch, which then has to hold only the plan and the SwiGLU terms: the reference's 2 * n * inter
// floats are enough for any n >= 1.
template <int CG, bool XL = false>
__global__ void __launch_bounds__(256) decode_gateup_kernel(DecodeArgs A) {
  const uint32_t slot = blockIdx.y;
  if (slot >= A.plan->n_slots) return;
  const uint32_t rt = blockIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t e = A.plan->expert[slot], mask = A.plan->tok_mask[slot], M = A.m_tokens;
  const uint32_t nst = A.hidden / kTileCols;
  // (XL: the activation loads go out before the weights, so waiting for them waits for nothing
  // else; an absent segment reloads segment 0, unused)
  float xv[XL ? 4 : 1][4];
  if constexpr (XL) {
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) segment_load(A.x, 0, 1, 0, q < nst ? q : 0u, xv[q]);
  }

  __shared__ uint32_t tbl[4 * kLut];
  __shared__ float part[4][2][CG][16][16];

  v4f acc[2][CG];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) acc[m][cg] = v4f{0.f, 0.f, 0.f, 0.f};

  // one column super-segment per wave (hidden <= 4096); its loads go out before the LDS table
  // is built, so both overlap
  const uint32_t S = wv;
  Unit ug, uu;
  if (S < nst) {
    const uint64_t tile = (uint64_t)rt * nst + S;
    load_unit(ug, plane_ptr(A, e, kGateCodes), plane_ptr(A, e, kGateFields), tile, lane);
    load_unit(uu, plane_ptr(A, e, kUpCodes), plane_ptr(A, e, kUpFields), tile, lane);
  }
  build_table(tbl, A.codebook);
  __shared__ __align__(16) uint8_t xl[XL ? kTerms * 4 * kTileCols : 16];
  __shared__ float red[4];
  if constexpr (XL) {
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
      if (q < nst) segment_split(xv[q], 0, q, A.hidden, xl, red);
      __syncthreads();  // (red is rewritten by the next segment)
    }
  }
  __syncthreads();
  if (S < nst) {
    const BSrc<CG> b = b_source<CG>(XL ? xl : A.xq, A.hidden, (uint64_t)S * kTileCols, lane, M, mask, A.zeros);
    // software pipeline: the table reads and B loads of step m+1 are issued before step m is
    // finished and multiplied; the scheduling barrier keeps the compiler from hoisting all
    // eight steps (register blow-up)
    uint32_t rg[8], ru[8];
    pin(ug);
    pin(uu);
    lookup_step(ug, tbl, 0, rg);
    lookup_step(uu, tbl, 0, ru);
    v8i bc[CG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) bc[cg] = b_step(b.p[cg], 0);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      uint32_t ng[8], nu[8];
      v8i bn[CG];
      if (m < 7) {
        pin(ug);
        pin(uu);
        lookup_step(ug, tbl, m + 1, ng);
        lookup_step(uu, tbl, m + 1, nu);
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) bn[cg] = b_step(b.p[cg], m + 1);
      }
      const v8i ag = finish_step(ug, m, rg), au = finish_step(uu, m, ru);
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        acc[0][cg] = mfma(ag, bc[cg], acc[0][cg]);
        acc[1][cg] = mfma(au, bc[cg], acc[1][cg]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (m < 7) {
#pragma unroll
        for (int i = 0; i < 8; ++i) { rg[i] = ng[i]; ru[i] = nu[i]; }
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) bc[cg] = bn[cg];
      }
    }
  }

  // accumulator lane l, element v = D[row 4*(l/16)+v][col l%16]
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
#pragma unroll
      for (int v = 0; v < 4; ++v) part[wv][m][cg][4 * (lane >> 4) + v][lane & 15] = acc[m][cg][v];
  __syncthreads();

  const uint32_t tid = threadIdx.x;
  if (tid < 16 * M) {
    const uint32_t r = tid & 15, t = tid >> 4;
    if ((mask >> t) & 1u) {
      const uint32_t cg = t / 5, col = (t % 5) * 3;
      const uint32_t nw = nst < 4 ? nst : 4;
      float s[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        float sum = 0.f;
        for (uint32_t q = 0; q < nw; ++q)  // super-segments in order, each at its own exponent
          sum += ldexpf(part[q][m][cg][r][col] + part[q][m][cg][r][col + 1] * 0.0625f +
                            part[q][m][cg][r][col + 2] * 0.00390625f,
                        -A.plan->x_sigma[t][q]);
        s[m] = sum;
      }
      const uint32_t row = rt * 16 + r;
      const float rg = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(plane_ptr(A, e, kGateRs))[row] << 16);
      const float ru = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(plane_ptr(A, e, kUpRs))[row] << 16);
      float g = s[0] * rg;
      float u = s[1] * ru;
      // SwiGLU with the asymmetric clamp: src/engine/ops.cpp:47-60
      const float L = A.limit;
      g = (L < g) ? L : g;
      const float lo = (-L < u) ? u : -L;
      u = (lo < L) ? lo : L;
      const float a = (g / (1.0f + expf(-g))) * u;
      uint32_t b0, b1, b2;
      split3(ldexpf(a, A.sigma_a), b0, b1, b2);
      uint8_t* dst = A.aq + ((uint64_t)(slot * M + t) * kTerms) * A.inter + row;
      dst[0] = (uint8_t)b0;
      dst[A.inter] = (uint8_t)b1;
      dst[2 * (uint64_t)A.inter] = (uint8_t)b2;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// down + weighted combine: one workgroup of 12 waves per 16-row tile of the output; the waves
// take the (slot, super-segment) units in turn (all of a batch-1 layer's twelve at once) and
// their per-token partials are summed in wave order.
// ------------------------------------------------------------------------------------------------
constexpr int kDownWaves = 12;

// SINGLE: every wave has at most one unit (units <= kDownWaves, e.g. batch 1: 6 experts x 2
// super-segments), which lets the compiler keep the loop-free body in registers.
template <int CG, bool SINGLE>
__global__ void __launch_bounds__(kDownWaves * 64) decode_down_kernel(DecodeArgs A) {
  const uint32_t rt = blockIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t M = A.m_tokens, ns = A.plan->n_slots;
  const uint32_t nst = A.inter / kTileCols, units = ns * nst;
  const uint32_t c = lane & 15, rg = lane >> 4;

  __shared__ uint32_t tbl[4 * kLut];
  __shared__ float part[kDownWaves][CG][16][16];

  float yacc[CG][4];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg)
#pragma unroll
    for (int v = 0; v < 4; ++v) yacc[cg][v] = 0.f;

  // the first unit's loads go out before the table is built; later units (batches with more
  // units than waves) are loaded at the top of their iteration, the other waves of the CU
  // covering the latency
  Unit cur;
  if (wv < units) {
    const uint32_t slot = wv / nst, S = wv % nst;
    const uint32_t e0 = A.plan->expert[slot];
    load_unit(cur, plane_ptr(A, e0, kDownCodes), plane_ptr(A, e0, kDownFields), (uint64_t)rt * nst + S, lane);
  }
  build_table(tbl, A.codebook);
  __syncthreads();

#pragma unroll 1
  for (uint32_t u = wv; u < (SINGLE ? (wv < units ? wv + 1 : 0) : units); u += kDownWaves) {
    const uint32_t slot = u / nst, S = u % nst;
    const uint32_t e = A.plan->expert[slot], mask = A.plan->tok_mask[slot];
    if (!SINGLE && u != wv)
      load_unit(cur, plane_ptr(A, e, kDownCodes), plane_ptr(A, e, kDownFields), (uint64_t)rt * nst + S, lane);
    const BSrc<CG> b = b_source<CG>(A.aq + (uint64_t)slot * M * kTerms * A.inter, A.inter,
                                    (uint64_t)S * kTileCols, lane, M, mask, A.zeros);
    const uint2 rsv = *reinterpret_cast<const uint2*>(plane_ptr(A, e, kDownRs) + (uint64_t)(rt * 16 + 4 * rg) * 2);
    __builtin_amdgcn_sched_barrier(0);
    v4f acc[CG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) acc[cg] = v4f{0.f, 0.f, 0.f, 0.f};
    uint32_t raw[8];
    pin(cur);
    lookup_step(cur, tbl, 0, raw);
    v8i bc[CG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) bc[cg] = b_step(b.p[cg], 0);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      uint32_t nraw[8];
      v8i bn[CG];
      if (m < 7) {
        pin(cur);
        lookup_step(cur, tbl, m + 1, nraw);
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) bn[cg] = b_step(b.p[cg], m + 1);
      }
      const v8i a = finish_step(cur, m, raw);
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) acc[cg] = mfma(a, bc[cg], acc[cg]);
      __builtin_amdgcn_sched_barrier(0);
      if (m < 7) {
#pragma unroll
        for (int i = 0; i < 8; ++i) raw[i] = nraw[i];
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) bc[cg] = bn[cg];
      }
    }
    const float rs[4] = {__uint_as_float(rsv.x << 16), __uint_as_float(rsv.x & 0xFFFF0000u),
                         __uint_as_float(rsv.y << 16), __uint_as_float(rsv.y & 0xFFFF0000u)};
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      const uint32_t t = cg * 5 + c / 3;
      const bool mine = c < 15 && (c % 3) == 0 && t < M && ((mask >> t) & 1u);
      const float wt = mine ? ldexpf(A.plan->w[slot][t], -A.sigma_a) : 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float val = combine_terms(acc[cg][v]);
        if (mine) yacc[cg][v] += val * rs[v] * wt;
      }
    }
  }

#pragma unroll
  for (int cg = 0; cg < CG; ++cg)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wv][cg][4 * rg + v][c] = yacc[cg][v];
  __syncthreads();
  const uint32_t tid = threadIdx.x;
  if (tid < 16 * M) {
    const uint32_t r = tid & 15, t = tid >> 4;
    const uint32_t cg = t / 5, col = (t % 5) * 3;
    float sum = 0.f;
    for (int q = 0; q < kDownWaves; ++q) sum += part[q][cg][r][col];
    float* dst = A.y + (uint64_t)t * A.y_ts + (uint64_t)(rt * 16 + r) * A.y_ds;
    *dst = A.accumulate ? *dst + sum : sum;
  }
}

// Workspace: [sync: fused-decode counters and flags, zero on first use][plan][zeros][xq][aq]
DecodeWs decode_ws(uint32_t M, uint32_t K, uint32_t hidden, uint32_t inter) {
  DecodeWs w;
  const uint64_t slots = (uint64_t)M * K;
  w.sync = 0;
  w.plan = a256(kSyncBytes);
  w.zeros = w.plan + a256(sizeof(DecodePlan));
  w.xq = w.zeros + 256;
  w.aq = w.xq + a256((uint64_t)M * kTerms * hidden);
  w.total = w.aq + a256(slots * M * kTerms * inter);
  return w;
}

}  // namespace affx

using namespace affx;

extern "C" {

size_t affx_decode_workspace_size(uint32_t m, uint32_t k, uint32_t hidden, uint32_t inter) {
  return (size_t)decode_ws(m, k, hidden, inter).total;
}

}  // extern "C"

namespace affx {

// Checks shared by the staged and fused paths; the workspace layout.
int decode_check(const affx_layer* L, uint32_t M, uint32_t K, const void* ws, size_t ws_bytes,
                 DecodeWs* lay) {
  if (!L || !ws || !L->base || !L->codebook) return set_error(AFFX_ERR_ARG, "ffn_decode: null pointer");
  if (M == 0 || M > kMaxTok || K == 0 || K > AFFX_MAX_TOPK)
    return set_error(AFFX_DECLINED, "ffn_decode: m_tokens must be 1..%d and top_k 1..%d (got %u, %u)",
                     kMaxTok, AFFX_MAX_TOPK, M, K);
  if (L->n_experts == 0 || L->n_experts > AFFX_MAX_EXPERTS)
    return set_error(AFFX_DECLINED, "ffn_decode: n_experts must be 1..%d", AFFX_MAX_EXPERTS);
  if (L->hidden % kTileCols || L->inter % kTileCols || L->hidden == 0 || L->inter == 0 ||
      L->hidden > 4 * kTileCols)
    return set_error(AFFX_DECLINED, "ffn_decode: hidden must be 1024..4096 and inter a multiple of "
                     "1024 (got %u, %u)", L->hidden, L->inter);
  if (!(L->swiglu_limit > 0.f) || L->swiglu_limit > 1e6f)
    return set_error(AFFX_DECLINED, "ffn_decode: needs a SwiGLU clamp limit in (0, 1e6]");
  *lay = decode_ws(M, K, L->hidden, L->inter);
  if (ws_bytes < lay->total)
    return set_error(AFFX_ERR_ARG, "ffn_decode: workspace %zu < %llu bytes", ws_bytes,
                     (unsigned long long)lay->total);
  uint64_t off9[9];
  const uint64_t stride = affx_expert_layout(L->hidden, L->inter, off9, nullptr);
  if (L->stride < stride) return set_error(AFFX_ERR_ARG, "ffn_decode: layer stride below expert size");
  return AFFX_OK;
}

int decode_sync_reset(void* ws, hipStream_t s) {
  return check_hip(hipMemsetAsync(ws, 0, kSyncBytes, s), "decode sync reset");
}

// decode_check, then the staged kernels' arguments.
int decode_setup(const affx_layer* L, uint32_t M, uint32_t K, void* ws, size_t ws_bytes,
                 DecodeArgs* A, DecodeWs* lay) {
  const int rc = decode_check(L, M, K, ws, ws_bytes, lay);
  if (rc) return rc;
  uint64_t off9[9];
  affx_expert_layout(L->hidden, L->inter, off9, nullptr);
  uint8_t* base = (uint8_t*)ws;
  A->base = (const uint8_t*)L->base;
  A->stride = L->stride;
  for (int i = 0; i < 9; ++i) A->off[i] = off9[i];
  A->hidden = L->hidden;
  A->inter = L->inter;
  A->m_tokens = M;
  A->codebook = (const uint32_t*)L->codebook;
  A->plan = (DecodePlan*)(base + lay->plan);
  A->xq = base + lay->xq;
  A->aq = base + lay->aq;
  A->zeros = base + lay->zeros;
  A->limit = L->swiglu_limit;
  // |SwiGLU| <= L * L under the clamp; scale so that it stays below 256 < 448
  A->sigma_a = 7 - ilogbf(L->swiglu_limit * L->swiglu_limit);
  A->n_tbl = 0;
  A->y = nullptr;
  A->y_ts = A->y_ds = 0;
  A->accumulate = 0;
  return AFFX_OK;
}

}  // namespace affx

extern "C" {

int affx_decode_prepare(const affx_layer* L, const float* x, uint64_t x_ts, uint64_t x_ds,
                        uint32_t M, const uint32_t* sel, const float* w, uint32_t K, void* ws,
                        size_t ws_bytes, void* stream) {
  DecodeArgs A;
  DecodeWs lay;
  if (!x || !sel || !w) return set_error(AFFX_ERR_ARG, "ffn_decode: null pointer");
  int rc = decode_setup(L, M, K, ws, ws_bytes, &A, &lay);
  if (rc) return rc;
  uint8_t* base = (uint8_t*)ws;
  hipLaunchKernelGGL(decode_prep_kernel, dim3(M * (L->hidden / kTileCols) + 1), dim3(256), 0,
                     (hipStream_t)stream, x, x_ts, x_ds,
                     M, sel, w, K, L->n_experts, L->hidden, (DecodePlan*)(base + lay.plan),
                     base + lay.xq, base + lay.zeros);
  return check_launch("decode_prep_kernel");
}

int affx_decode_gateup(const affx_layer* L, uint32_t M, uint32_t K, void* ws, size_t ws_bytes,
                       void* stream) {
  DecodeArgs A;
  DecodeWs lay;
  int rc = decode_setup(L, M, K, ws, ws_bytes, &A, &lay);
  if (rc) return rc;
  const uint32_t max_slots = M * K < L->n_experts ? M * K : L->n_experts;
  const dim3 g(L->inter / kTileRows, max_slots);
  if (M <= 5) hipLaunchKernelGGL(decode_gateup_kernel<1>, g, dim3(256), 0, (hipStream_t)stream, A);
  else hipLaunchKernelGGL(decode_gateup_kernel<2>, g, dim3(256), 0, (hipStream_t)stream, A);
  return check_launch("decode_gateup_kernel");
}

int affx_decode_down(const affx_layer* L, uint32_t M, uint32_t K, float* y, uint64_t y_ts,
                     uint64_t y_ds, int accumulate, void* ws, size_t ws_bytes, void* stream) {
  DecodeArgs A;
  DecodeWs lay;
  if (!y) return set_error(AFFX_ERR_ARG, "ffn_decode: null pointer");
  int rc = decode_setup(L, M, K, ws, ws_bytes, &A, &lay);
  if (rc) return rc;
  A.y = y;
  A.y_ts = y_ts;
  A.y_ds = y_ds;
  A.accumulate = accumulate;
  const dim3 g(L->hidden / kTileRows), blk(kDownWaves * 64);
  // the number of units is known on the device only; M*K distinct experts bound it
  const uint32_t max_units = (M * K < L->n_experts ? M * K : L->n_experts) * (L->inter / kTileCols);
  hipStream_t st = (hipStream_t)stream;
  if (M <= 5) {
    if (max_units <= (uint32_t)kDownWaves) hipLaunchKernelGGL((decode_down_kernel<1, true>), g, blk, 0, st, A);
    else hipLaunchKernelGGL((decode_down_kernel<1, false>), g, blk, 0, st, A);
  } else {
    hipLaunchKernelGGL((decode_down_kernel<2, false>), g, blk, 0, st, A);
  }
  return check_launch("decode_down_kernel");
}

int affx_decode_staged(const affx_layer* L, const float* x, uint64_t x_ts, uint64_t x_ds,
                           uint32_t M, const uint32_t* sel, const float* w, uint32_t K, float* y,
                           uint64_t y_ts, uint64_t y_ds, int accumulate, void* ws,
                           size_t ws_bytes, void* stream) {
  if (!y) return set_error(AFFX_ERR_ARG, "ffn_decode: null pointer");
  int rc = affx_decode_prepare(L, x, x_ts, x_ds, M, sel, w, K, ws, ws_bytes, stream);
  if (rc) return rc;
  rc = affx_decode_gateup(L, M, K, ws, ws_bytes, stream);
  if (rc) return rc;
  return affx_decode_down(L, M, K, y, y_ts, y_ds, accumulate, ws, ws_bytes, stream);
}

// expert_ffn_hip's arguments (src/gpu/expert_kernel_hip.h:273): one token through n experts given
// as a host array of per-matrix device pointers, out += sum_k weights[k] * FFN_k(x). The staged
// kernels with the plane-pointer table in their arguments and route k = expert k; no cross-workgroup
// state, so the caller's scratch needs no clearing. Its layout: [plan][zeros][xq][aq].
int affx_expert_ffn(const affx_device_expert* experts, const float* weights, uint32_t n,
                    const void* codebook, const float* x, float swiglu_limit, float* scratch, float* out,
                    void* stream) {
  if (n == 0) return AFFX_OK;
  if (!experts || !weights || !codebook || !x || !scratch || !out)
    return set_error(AFFX_ERR_ARG, "expert_ffn: null pointer");
  if (n > kTblMax) return set_error(AFFX_DECLINED, "expert_ffn: at most %u experts per call (got %u)", kTblMax, n);
  const uint32_t inter = experts[0].gate.rows, hidden = experts[0].gate.cols;
  if (hidden % kTileCols || inter % kTileCols || hidden == 0 || inter == 0 || hidden > 4 * kTileCols)
    return set_error(AFFX_DECLINED, "expert_ffn: hidden must be 1024..4096 and inter a multiple of 1024 "
                     "(got %u, %u)", hidden, inter);
  if (!(swiglu_limit > 0.f) || swiglu_limit > 1e6f)
    return set_error(AFFX_DECLINED, "expert_ffn: needs a SwiGLU clamp limit in (0, 1e6]");
  DecodeArgs A{};
  A.n_tbl = n;
  for (uint32_t k = 0; k < n; ++k) {
    const affx_matrix* m[3] = {&experts[k].gate, &experts[k].up, &experts[k].down};
    for (int i = 0; i < 3; ++i) {
      const uint32_t rows = i < 2 ? inter : hidden, cols = i < 2 ? hidden : inter;
      if (m[i]->rows != rows || m[i]->cols != cols || !m[i]->codes || !m[i]->fields || !m[i]->rscales)
        return set_error(AFFX_ERR_ARG, "expert_ffn: expert %u matrix %d is %ux%u, expected %ux%u with planes", k, i,
                         m[i]->rows, m[i]->cols, rows, cols);
      A.tbl[k][3 * i + 0] = (const uint8_t*)m[i]->codes;
      A.tbl[k][3 * i + 1] = (const uint8_t*)m[i]->fields;
      A.tbl[k][3 * i + 2] = (const uint8_t*)m[i]->rscales;
    }
  }
  // scratch: the reference's contract is 2 * n * inter floats. It holds the plan (only its first
  // n slots' weights: the weight table is the plan's last member), the zero row and the SwiGLU
  // terms; the activation terms are made in each gate/up workgroup's LDS.
  const uint64_t plan = 0, zeros = a256(offsetof(DecodePlan, w) + sizeof(float) * kMaxTok * n), aq = zeros + 256;
  const uint64_t need = aq + 3ull * n * inter, have = 8ull * n * inter;
  if (need > have)
    return set_error(AFFX_DECLINED, "expert_ffn: needs %llu bytes of scratch, the 2 * n * inter floats hold %llu",
                     (unsigned long long)need, (unsigned long long)have);
  uint8_t* ws = (uint8_t*)scratch;
  A.base = nullptr;
  A.stride = 0;
  A.hidden = hidden;
  A.inter = inter;
  A.m_tokens = 1;
  A.codebook = (const uint32_t*)codebook;
  A.plan = (const DecodePlan*)(ws + plan);
  A.xq = nullptr;
  A.x = x;
  A.aq = ws + aq;
  A.zeros = ws + zeros;
  A.limit = swiglu_limit;
  A.sigma_a = 7 - ilogbf(swiglu_limit * swiglu_limit);
  A.y = out;
  A.y_ts = hidden;
  A.y_ds = 1;
  A.accumulate = 1;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(decode_prep_kernel, dim3(hidden / kTileCols + 1), dim3(256), 0, st, x, (uint64_t)hidden,
                     (uint64_t)1, 1u, (const uint32_t*)nullptr, weights, n, n, hidden, (DecodePlan*)(ws + plan),
                     (uint8_t*)nullptr, ws + zeros);
  int rc = check_launch("decode_prep_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((decode_gateup_kernel<1, true>), dim3(inter / kTileRows, n), dim3(256), 0, st, A);
  if ((rc = check_launch("decode_gateup_kernel"))) return rc;
  const uint32_t units = n * (inter / kTileCols);
  if (units <= (uint32_t)kDownWaves)
    hipLaunchKernelGGL((decode_down_kernel<1, true>), dim3(hidden / kTileRows), dim3(kDownWaves * 64), 0, st, A);
  else
    hipLaunchKernelGGL((decode_down_kernel<1, false>), dim3(hidden / kTileRows), dim3(kDownWaves * 64), 0, st, A);
  return check_launch("decode_down_kernel");
}

}  // extern "C"
