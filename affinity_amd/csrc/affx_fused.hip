// Fused decode of one MoE layer (M <= 8 tokens): one launch runs routing plan, activation split,
// gate/up + SwiGLU and down + weighted combine.
//
// One workgroup of 12 waves per CU, all resident at once (the grid never exceeds what the device
// holds concurrently). Every workgroup
//   1. builds the routing plan itself (distinct experts ascending, token masks, summed weights),
//   2. issues the HBM loads of its gate/up tiles AND of its first down tile right away, so the
//      down weights stream in while gate/up is computed,
//   3. splits the activation into three E4M3 terms in LDS (hardware fp8 conversion) and stages
//      the codebook in LDS as KC interleaved copies (lane-fixed copy: gathers from 64 lanes spread
//      over the 64 banks instead of colliding at random),
//   4. computes its gate/up items (16 rows x all columns of one expert; wave = 1024-column
//      segment), sums the segments in fixed order, applies SwiGLU and writes the result as E4M3
//      terms (aq) to global memory with device-coherent stores, drains them, and adds its item
//      count to one agent-scope counter; the add that completes the count clears it and raises
//      one release flag per down-phase workgroup (a 128-byte line each),
//   5. waits (bounded spin) on its own flag, clears it, then computes one 16-row tile of the
//      output from its (expert, segment) down units and writes y.
// Counter and flags are zero again when the launch ends, so the workspace is reusable by the next
// launch on the stream without a memset (graph-capture safe).
//
// Batch 1 (the one-pass kernel, SINGLE) replaces step 4's counter and flags: each workgroup stores
// the launch's epoch into its own dword of eight publish-flag copies, and a down-phase workgroup
// polls the copy of its XCD until every gate/up workgroup's dword shows the epoch; the last
// workgroup then advances the epoch word. Nothing is cleared, so this form too needs no memset.
//
// Reference counterparts: the routed-expert batch hook ExpertFfnBatch (src/engine/model.h:658-666,
// called at src/engine/model.cpp:1663-1664, bound to run_batch_device at tools/affinity.cpp:
// 1218-1236) and the per-token expert_ffn_hip (src/gpu/expert_kernel.hip:2737-2808), with the
// routing plan of moe_plan (src/gpu/moe_plan.hip).
#include <mutex>

#include "affx_lut.h"

namespace affx {

constexpr int kFW = 12;                      // waves per workgroup
constexpr int kPollUnitsMax = kFW;           // down units of the one-pass kernel: one per wave
constexpr int kFT = kFW * 64;                // threads per workgroup
constexpr int kXqChunk = 272;                // LDS bytes of one 256-column chunk of an xq row
constexpr int kXqRow = 16 * kXqChunk + 64;   // LDS bytes of one (token, term) row, hidden <= 4096
constexpr uint32_t kSpinLimit = 1u << 22;    // polls (~2^22 x 128 cycles ~ 0.2 s) before giving up
constexpr int kPlanRoutes = AFFX_MAX_DECODE_TOKENS * AFFX_MAX_TOPK;  // 128
// How the kernel reads x (element (t, h) at x[t * xts + h * xds]):
//  kXStrided     any strides, four loads per four elements;
//  kXTokenMajor  xds = 1, 16-byte aligned rows: 16-byte loads;
//  kXDimMajor    xts = 1 (the engine's dim-major batch arena, rows of xds >= M floats), xds a
//                multiple of 4 and x 16-byte aligned: read one token at a time, a pair's
//                elements would sit xds * 4 bytes apart and every load instruction would touch
//                64 cache lines, so the kernel reads whole 16-byte row pieces of 4 tokens.
// A kernel per form: with the forms as branches of one kernel, the compiler shared the load
// instructions between them (the token-major form lost its 16-byte loads) or, kept apart, waited
// for every load in flight where the branches joined.
enum XForm { kXStrided = 0, kXTokenMajor = 1, kXDimMajor = 2 };

struct FusedArgs {
  const uint8_t* base;
  uint64_t stride;
  uint64_t off[9];
  uint32_t hidden, inter, M, K, n_experts, n_wg;
  const uint32_t* codebook;
  const float* x;
  uint64_t xts, xds;
  const uint32_t* sel;
  const float* w;
  uint8_t* aq;          // [slot][M][3][inter]
  const uint8_t* zeros; // 256 zero bytes (B source of unused down columns)
  uint32_t* sync;       // [0] gate/up items published, [2] error bits; release flags from byte 256
  float* y;
  uint64_t yts, yds;
  int accumulate;
  float limit;
  int32_t sigma_a;
  uint32_t spin_limit;  // polls of the release flag before a waiter gives up (sets error bit 0)
};

// Dynamic LDS layout in bytes (host and device agree): activation terms, zero run, partial sums,
// plan. The codebook copies are the kernel's one static LDS array (at address 0, so a table
// address needs no base add).
struct FusedLds {
  uint32_t xq, zero, part, plan, count, total;
};

__host__ __device__ inline FusedLds fused_lds(uint32_t M) {
  FusedLds L;
  L.xq = 0;
  L.zero = L.xq + 3u * M * kXqRow;
  L.part = L.zero + 256u;
  const uint32_t part_bytes = (uint32_t)kFW * 2u * 16u * M * 4u;  // gate/up [wave][mat][row][tok]
  L.plan = L.part + part_bytes;
  // slot_expert[128] slot_mask[128] rs[12][32] sigma[32] slot_w[128][M] slot_tok[128]
  L.count = L.plan + (3u * kPlanRoutes + kFW * 32u + 32u) * 4u + kPlanRoutes * M * 4u;
  // four words: [0] waves counted in after the set-up (batch 1), [1] the slot count (rounds
  // kernels, from the plan wave), [2] waves done with the current round's epilogue (rounds kernels)
  L.total = L.count + 16u;
  return L;
}

// B operand of one MFMA step from the LDS activation rows: two 16-byte reads.
__device__ __forceinline__ v8i b_step_lds(const uint8_t* p, int m) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(p + 32 * m);
  const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 32 * m + 16);
  v8i v;
  v[0] = (int)lo[0]; v[1] = (int)lo[1]; v[2] = (int)lo[2]; v[3] = (int)lo[3];
  v[4] = (int)hi[0]; v[5] = (int)hi[1]; v[6] = (int)hi[2]; v[7] = (int)hi[3];
  return v;
}

// The gate and up units of one wave tile, loaded in the order the MFMA steps need them (both
// field runs, then code chunk j of gate and of up for j = 0..4): loads complete in issue order, so
// step m only waits for the chunks it reads. The scheduling barriers keep that order.
__device__ __forceinline__ void load_pair(Unit& g, Unit& u, const uint8_t* gc, const uint8_t* gf,
                                          const uint8_t* uc, const uint8_t* uf, uint64_t tile, uint32_t lane) {
  const uint32_t* gfp = reinterpret_cast<const uint32_t*>(gf + tile * kTileFieldBytes + lane * 12);
  const uint32_t* ufp = reinterpret_cast<const uint32_t*>(uf + tile * kTileFieldBytes + lane * 12);
  g.f[0] = __builtin_nontemporal_load(gfp);
  g.f[1] = __builtin_nontemporal_load(gfp + 1);
  g.f[2] = __builtin_nontemporal_load(gfp + 2);
  u.f[0] = __builtin_nontemporal_load(ufp);
  u.f[1] = __builtin_nontemporal_load(ufp + 1);
  u.f[2] = __builtin_nontemporal_load(ufp + 2);
  __builtin_amdgcn_sched_barrier(0);
  const uint8_t* gcp = gc + tile * kTileCodeBytes + lane * 16;
  const uint8_t* ucp = uc + tile * kTileCodeBytes + lane * 16;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gcp + j * 1024));
    const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ucp + j * 1024));
    g.c[4 * j] = a[0]; g.c[4 * j + 1] = a[1]; g.c[4 * j + 2] = a[2]; g.c[4 * j + 3] = a[3];
    u.c[4 * j] = b[0]; u.c[4 * j + 1] = b[1]; u.c[4 * j + 2] = b[2]; u.c[4 * j + 3] = b[3];
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Compacted columns (one 16-column group serving up to eight tokens): in pass p over a slot's
// weights, column c < 15 holds term c % 3 of the slot's (5p + c/3)-th token in ascending order.
// tl: the slot's tokens in that order, four bits each; nt: their count. Returns whether the
// column is used; t is then its token.
__device__ __forceinline__ bool cmp_column(uint32_t tl, uint32_t nt, uint32_t p, uint32_t c, uint32_t& t) {
  const uint32_t j = 5u * p + c / 3u;
  t = (tl >> ((4u * j) & 31u)) & 15u;
  return c < 15u && j < nt;
}

// Packed ascending token list of a token mask (at most eight tokens: four bits each).
__device__ __forceinline__ uint32_t token_list(uint32_t mask) {
  uint32_t tl = 0, k = 0;
#pragma unroll
  for (int b = 0; b < AFFX_MAX_DECODE_TOKENS; ++b)
    if ((mask >> b) & 1u) {
      tl |= (uint32_t)b << (4u * k);
      ++k;
    }
  return tl;
}

// value of the three E4M3 term columns c, c+1, c+2 (valid in lanes whose column is a multiple of 3)
__device__ __forceinline__ float fused_terms(float d) {
  const float d1 = row_shl<1>(d), d2 = row_shl<2>(d);  // (DPP row shifts)
  return d + d1 * 0.0625f + d2 * 0.00390625f;
}


// maximum over the wave, wave-uniform: DPP row shifts leave each 16-lane row's maximum in its
// last lane, then the four rows' last lanes are combined (no LDS round trips)
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, row_shr<1>(v));
  v = fmaxf(v, row_shr<2>(v));
  v = fmaxf(v, row_shr<4>(v));
  v = fmaxf(v, row_shr<8>(v));
  const int b = __float_as_int(v);
  return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 15)), __int_as_float(__builtin_amdgcn_readlane(b, 31))),
               fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 47)), __int_as_float(__builtin_amdgcn_readlane(b, 63))));
}

// ------------------------------------------------------------------------------------------------
// The kernel. CG: 16-column groups of the MFMA B operand (five tokens each; one). KC: codebook
// copies. MAXM: largest M this instantiation serves (sizes the per-thread activation registers).
// With MAXM > 5 the columns are compacted: each slot's tokens fill the group pass by pass
// (cmp_column), so a slot serving five tokens or fewer (almost all of them in a decode batch)
// costs one MFMA per weight fragment. The down weights of each wave's first unit are requested
// before the wait for the SwiGLU output. SINGLE: at most
// one gate/up item and one down unit (per output tile) per wave, which keeps those two phases
// loop-free (batch 1). ROT: the codebook copies include the rotated tables (one VALU op less
// per code, twice the LDS). XF: how x is read (an XForm; the host picks it from the strides).
// ------------------------------------------------------------------------------------------------
template <int CG, int KC, int MAXM, bool SINGLE, bool ROT, int XF>
__global__ void __launch_bounds__(kFT) decode_fused_kernel(FusedArgs A) {
  AFFX_DYN_LDS(lds);
  // One column group: M <= 5 in fixed columns, M > 5 in compacted ones (two fixed groups of five
  // tokens, the earlier form for M > 5, cost a second MFMA per weight fragment and did not leave
  // the registers for the whole down B operand).
  static_assert(CG == 1, "the fused decode holds one column group");
  // the first down unit is loaded while gate/up runs (one column group leaves the registers)
  constexpr bool PREF = true;
  // compacted columns: a slot with more than five tokens takes a second pass over its weights
  // (decoded again from the registers that hold them)
  constexpr bool CMP = MAXM > 5;
  const uint32_t tid = threadIdx.x, lane = tid & 63, g = blockIdx.x;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const uint32_t M = A.M, K = A.K, R = M * K;
  const uint32_t nst = A.hidden / kTileCols, nsi = A.inter / kTileCols;
  const FusedLds L = fused_lds(M);
  __shared__ __align__(16) uint32_t lut_s[Lut<KC, ROT>::kDwords];
  const uint8_t* lut = reinterpret_cast<const uint8_t*>(lut_s);
  // (the finish computes each block's sign mask and exponent add itself: two registers fewer per
  // block in flight than the block table's, which this kernel's register budget needs)
  const uint8_t* btbl = nullptr;
  uint8_t* xq = lds + L.xq;
  uint8_t* zero_l = lds + L.zero;
  float* part = reinterpret_cast<float*>(lds + L.part);
  uint32_t* slot_expert = reinterpret_cast<uint32_t*>(lds + L.plan);
  uint32_t* slot_mask = slot_expert + kPlanRoutes;
  float* rs_l = reinterpret_cast<float*>(slot_mask + kPlanRoutes);  // [group][gate 16 | up 16]
  int32_t* sigma_l = reinterpret_cast<int32_t*>(rs_l + kFW * 32);
  float* slot_w = reinterpret_cast<float*>(sigma_l + 32);
  // (compacted columns) each slot's tokens in ascending order, four bits each
  uint32_t* slot_tok = reinterpret_cast<uint32_t*>(slot_w + kPlanRoutes * M);

  AFFX_TRACE_INIT;
  AFFX_TRACE(0);
  // batch 1: the count of waves whose share of the LDS set-up (plan, activation terms, codebook
  // copies) is written; it replaces the workgroup barrier before gate/up (step 3)
  uint32_t* parts_in = reinterpret_cast<uint32_t*>(lds + L.count);
  if constexpr (SINGLE) {
    if (tid == 0) *parts_in = 0u;
    __syncthreads();
  } else {
    if (tid == 0) parts_in[2] = 0u;  // epilogue waves done (the set-up barrier publishes the zero)
  }
  // ---- 1. the small loads first (routes, then codebook and activation: loads complete in issue
  // order, so waiting for them never waits for the weight stream issued after them); every wave
  // dedupes the routes itself (registers only) so that it can issue its weight loads as soon as
  // the routes arrive, with no barrier in between.
  // Batch 1: the launch epoch, requested before anything else (needed only at the publish; loads
  // complete in issue order, so no earlier wait covers it).
  uint32_t ep_raw = 0;
  if constexpr (SINGLE) ep_raw = __hip_atomic_load(&A.sync[kEpochWord], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Routes r = lane + 64 h. Slots are the distinct experts in order of first occurrence.
  uint32_t e[2];
  float wr[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t r = lane + 64u * h, rr = r < R ? r : 0u;
    e[h] = A.sel[rr];
    wr[h] = A.w[rr];
  }
  // codebook entries tid, tid + 768, tid + 1536; activation pairs p = wv + 12 j (token p / nst,
  // 1024-column segment p % nst; an absent pair reloads pair 0, unused)
  uint32_t cbv[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const uint32_t ce = tid + (uint32_t)i * kFT;
    cbv[i] = A.codebook[ce < 2048u ? ce : 0u];
  }
  constexpr int NP = (MAXM * 4 + kFW - 1) / kFW;
  // kXDimMajor: each wave takes a unit of four tokens of one 1024-column segment instead of a
  // (token, segment) pair; each lane reads the 16-byte row pieces (tokens 4 g4 .. 4 g4 + 3) of its
  // four consecutive rows per 256-column chunk, which leaves it the same four consecutive
  // columns of each token that a pair gives it.
  constexpr int NX = XF == kXDimMajor ? 16 : NP * 4;
  float4 xr[NX];  // pairs: xr[4 j + i]; units: xr[4 i + r]
  const uint32_t xquads = (M + 3) / 4;
  {
    // element offsets in 32 bits (the host sends larger arenas to the staged launches)
    const uint32_t xts = (uint32_t)A.xts, xds = (uint32_t)A.xds;
    if constexpr (XF == kXTokenMajor) {
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const uint32_t p0 = wv + (uint32_t)j * kFW, p = p0 < M * nst ? p0 : 0u;
        const uint32_t t = p / nst, Sx = p % nst;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          xr[4 * j + i] = *reinterpret_cast<const float4*>(A.x + (t * xts + Sx * kTileCols + 4 * (lane + 64 * i)));
      }
    } else if constexpr (XF == kXDimMajor) {
      if (wv < xquads * nst) {
        const uint32_t g4 = wv / nst, Sx = wv % nst;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t h = Sx * kTileCols + 256u * i + 4u * lane + r;
            xr[4 * i + r] = *reinterpret_cast<const float4*>(A.x + (h * xds + 4u * g4));
          }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const uint32_t p0 = wv + (uint32_t)j * kFW, p = p0 < M * nst ? p0 : 0u;
        const uint32_t t = p / nst, Sx = p % nst;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t o = t * xts + (Sx * kTileCols + 4 * (lane + 64 * i)) * xds;
          xr[4 * j + i] = make_float4(A.x[o], A.x[o + xds], A.x[o + 2 * xds], A.x[o + 3 * xds]);
        }
      }
    }
  }
  AFFX_TRACE(8);
  // dedupe: slots are the distinct experts in order of first occurrence (ids outside the layer
  // are ignored, as in the staged path). One pass per distinct expert over the wave's routes
  // (route r = lane + 64 h): the lowest route not yet assigned names the next slot's expert, a
  // ballot finds all its routes. Lane s of se[0] (se[1]) then holds the expert of slot s
  // (s + 64).
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t r = lane + 64u * h;
    // (absent routes OR in all ones: a select on r < R lets the compiler move the route load
    // into a branch that then waits for every load in flight)
    const uint32_t v = e[h] | (r < R ? 0u : ~0u);
    e[h] = v < A.n_experts ? v : ~0u;
  }
  // Rounds kernels: only the plan wave (wave 0) finds every slot. The others stop once they know
  // the slot of their round-0 item, issue its loads, and take the rest from the plan in LDS after
  // the set-up barrier (with some 44 distinct experts at M = 8, every wave otherwise ran 44 ballot
  // rounds before it requested its weights, the three waves of a SIMD sharing its issue).
  const uint32_t rt_per = A.inter / kTileRows;          // gate/up row tiles per expert
  const uint32_t groups = kFW / nst;                    // items in flight per workgroup
  const uint32_t q = wv / nst, S = wv % nst;            // this wave: group, column segment
  const uint32_t item0 = g + A.n_wg * q;                // this wave's round-0 item (if there is one)
  const uint32_t stop_at = (SINGLE || wv == 0) ? ~0u : item0 / rt_per + 1u;
  uint32_t se[2] = {~0u, ~0u};
  uint32_t rslot[2] = {~0u, ~0u};  // slot of route lane + 64 h
  uint32_t ns = 0;
  if (!SINGLE && MAXM > 1 && wv == 0 && M >= 2u) {
    // The plan wave of the rounds kernels finds every slot at once (the ballot loop below takes one
    // round per slot: some 4 us at M = 8, on the path to the set-up barrier). The LDS of the
    // partial sums, unused until the rounds (1536 M bytes: room for 384 M experts), holds per
    // expert its lowest route, then its slot. A route is its expert's first occurrence where it is
    // that lowest route; its slot is its rank among the first occurrences.
    uint32_t* fr = reinterpret_cast<uint32_t*>(lds + L.part);
    for (uint32_t i = lane; i < A.n_experts; i += 64u) fr[i] = ~0u;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (e[h] != ~0u) atomicMin(&fr[e[h]], lane + 64u * h);
    __builtin_amdgcn_wave_barrier();
    bool lead[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) lead[h] = e[h] != ~0u && fr[e[h]] == lane + 64u * h;
    const uint64_t b0 = __ballot(lead[0]), b1 = __ballot(lead[1]);
    const uint32_t n0 = (uint32_t)__builtin_popcountll(b0);
    const uint32_t rank[2] = {
        __builtin_amdgcn_mbcnt_hi((uint32_t)(b0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b0, 0u)),
        __builtin_amdgcn_mbcnt_hi((uint32_t)(b1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b1, n0))};
    ns = n0 + (uint32_t)__builtin_popcountll(b1);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (lead[h]) {
        fr[e[h]] = rank[h];
        slot_expert[rank[h]] = e[h];
      }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int h = 0; h < 2; ++h) rslot[h] = e[h] != ~0u ? fr[e[h]] : ~0u;
    se[0] = lane < ns ? slot_expert[lane] : ~0u;
    se[1] = lane + 64u < ns ? slot_expert[lane + 64u] : ~0u;
  } else {
    uint64_t pend0 = __ballot(e[0] != ~0u), pend1 = __ballot(e[1] != ~0u);
    while ((pend0 | pend1) && (SINGLE || ns < stop_at)) {
      const uint32_t ex = pend0 ? __builtin_amdgcn_readlane(e[0], (uint32_t)__builtin_ctzll(pend0))
                                : __builtin_amdgcn_readlane(e[1], (uint32_t)__builtin_ctzll(pend1));
      pend0 &= ~__ballot(e[0] == ex);
      pend1 &= ~__ballot(e[1] == ex);
      rslot[0] = e[0] == ex ? ns : rslot[0];
      rslot[1] = e[1] == ex ? ns : rslot[1];
      if (lane == (ns & 63u)) {
        if (ns < 64u) se[0] = ex;
        else se[1] = ex;
      }
      ++ns;
    }
  }
  AFFX_TRACE(12);
  // expert of slot s (s wave-uniform): from the registers, or (rounds kernels, once the set-up
  // barrier has passed) from the plan in LDS
  bool plan_in_lds = false;
  auto slot_expert_of = [&](uint32_t s) -> uint32_t {
    if (!SINGLE && plan_in_lds) return __builtin_amdgcn_readfirstlane(slot_expert[s]);
    return s < 64u ? __builtin_amdgcn_readlane(se[0], s) : __builtin_amdgcn_readlane(se[1], s - 64u);
  };
  // the counts that follow from the number of slots (rounds kernels: set again after the set-up
  // barrier, when every wave knows it)
  uint32_t NI, my_items, rounds, NU;
  auto set_counts = [&]() {
    NI = ns * rt_per;                                   // gate/up items of the layer
    my_items = g < NI ? (NI - g + A.n_wg - 1) / A.n_wg : 0;
    rounds = (my_items + groups - 1) / groups;
    NU = ns * nsi;                                      // down units per output tile
  };
  set_counts();
  const uint32_t dtiles = A.hidden / kTileRows;
  const uint32_t copy4 = ((lane >> 1) & (KC - 1)) * 4u;

  // ---- 2. loads: gate/up pair of round 0 (+ its row scales), and the first down unit (+ row
  // scales) when round 0 is the last; the compute below waits for them
  Unit ug, uu, ud;
  uint32_t rs_gu = 0;  // bf16 row scale: lanes 0-15 gate rows, 16-31 up rows (segment-0 waves)
  uint2 rs_d = {0u, 0u};
  auto gu_item = [&](uint32_t rho) -> uint32_t {
    const uint32_t k = rho * groups + q;
    return (q < groups && k < my_items) ? g + A.n_wg * k : ~0u;
  };
  // unconditional loads (an absent item or unit reads expert 0's first tile, never used): the
  // wait-count tracking then sees straight-line code and waits for exactly what each step needs
  // rounds kernels: the next round's gate/up pair is requested step by step during this round's
  // MFMA steps, each part into the registers the steps before it left dead (a ring), so the
  // requests reach the vector memory address unit spread over the round instead of as one burst
  // after it (which the unit took about 2 us per round to accept, with every wave stalled on it
  // and the decode idle); the row scales then come first, so that the wait for them at the start
  // of a round covers no weights
  constexpr bool RING = !SINGLE;
  auto load_gu = [&](uint32_t item) {
    const bool ok = item != ~0u;
    const uint32_t slot = ok ? item / rt_per : 0u, rt = ok ? item % rt_per : 0u;
    const uint32_t e = ok ? slot_expert_of(slot) : 0u;
    const uint8_t* ex = A.base + (uint64_t)e * A.stride;
    const uint64_t tile = ok ? (uint64_t)rt * nst + S : 0u;
    auto row_scale = [&]() {
      return reinterpret_cast<const uint16_t*>(ex + A.off[lane < 16 ? kGateRs : kUpRs])[rt * 16 + (lane & 15)];
    };
    if constexpr (RING) {
      rs_gu = row_scale();
      __builtin_amdgcn_sched_barrier(0);
    }
    load_pair(ug, uu, ex + A.off[kGateCodes], ex + A.off[kGateFields], ex + A.off[kUpCodes],
              ex + A.off[kUpFields], tile, lane);
    if constexpr (!RING) rs_gu = row_scale();
    __builtin_amdgcn_sched_barrier(0);
  };
  auto load_down = [&](bool ok, uint32_t td, uint32_t u) {
    const uint32_t slot = ok ? u / nsi : 0u, S2 = ok ? u % nsi : 0u;
    const uint32_t e = ok ? slot_expert_of(slot) : 0u;
    const uint8_t* ex = A.base + (uint64_t)e * A.stride;
    const uint32_t tdd = ok ? td : 0u;
    load_unit_ordered(ud, ex + A.off[kDownCodes], ex + A.off[kDownFields], (uint64_t)tdd * nsi + S2, lane);
    rs_d = *reinterpret_cast<const uint2*>(ex + A.off[kDownRs] + (uint64_t)(tdd * 16 + 4 * (lane >> 4)) * 2);
    __builtin_amdgcn_sched_barrier(0);
  };
  bool has_down = g < dtiles && wv < NU;
  // the waves that write the SwiGLU output drain their memory counter before the release
  const uint32_t epi_waves = (groups * 16 * M + 63) / 64;
  // (batch 1 issues them after its share of the LDS set-up, step 3)
  if constexpr (!SINGLE) load_gu(q < groups && item0 / rt_per < ns ? item0 : ~0u);
  AFFX_TRACE(13);
  AFFX_TRACE(2);

  // ---- the plan for the epilogue and the down phase: expert of every slot, token masks, and
  // per (slot, token) the summed weight of the token's routes to the slot, added in route order
  // as the staged plan does (lane t walks token t's routes; no two lanes touch the same entry).
  // Batch 1: the last wave writes it (the first waves split the activation; with both on wave 0
  // that wave's share of the set-up was the last to finish); larger batches: wave 0.
  if (wv == (SINGLE ? (uint32_t)kFW - 1u : 0u)) {
    if (lane == 0) parts_in[1] = ns;  // (rounds kernels: the slot count for the other waves)
    if (lane < ns) slot_expert[lane] = se[0];
    if (lane + 64u < ns) slot_expert[lane + 64u] = se[1];
    for (uint32_t i = lane; i < ns * M; i += 64u) slot_w[i] = 0.f;
    for (uint32_t i = lane; i < ns; i += 64u) slot_mask[i] = 0u;
    __builtin_amdgcn_wave_barrier();
    for (uint32_t j = 0; j < K; ++j) {
      const uint32_t r = lane * K + j;              // route j of token `lane`
      const uint32_t src = (r & 63u) * 4u;          // bpermute byte index
      const uint32_t s0 = (uint32_t)__builtin_amdgcn_ds_bpermute((int)src, (int)rslot[0]);
      const uint32_t s1 = (uint32_t)__builtin_amdgcn_ds_bpermute((int)src, (int)rslot[1]);
      const float w0 = __int_as_float(__builtin_amdgcn_ds_bpermute((int)src, __float_as_int(wr[0])));
      const float w1 = __int_as_float(__builtin_amdgcn_ds_bpermute((int)src, __float_as_int(wr[1])));
      const uint32_t sl = r < 64u ? s0 : s1;
      if (lane < M && sl != ~0u) {
        slot_w[sl * M + lane] += r < 64u ? w0 : w1;
        atomicOr(&slot_mask[sl], 1u << lane);
      }
    }
    if constexpr (CMP) {
      // (the masks are complete: one wave's LDS operations take effect in order)
      __builtin_amdgcn_wave_barrier();
      for (uint32_t i = lane; i < ns; i += 64u) slot_tok[i] = token_list(slot_mask[i]);
    }
  }
  AFFX_TRACE(9);

  // ---- 3. activation terms and codebook copies into LDS, from the registers loaded up front:
  // a pair's maximum (wave reduction) fixes its exponent, then three E4M3 terms per element
  auto stage_pair = [&](uint32_t t, uint32_t Sx, float4 v0, float4 v1, float4 v2, float4 v3) {
    const float4 v[4] = {v0, v1, v2, v3};
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    mx = wave_max(mx);
    // amax * 2^sigma in [128, 256): below E4M3's 448
    const int sigma = mx > 0.f ? 7 - ilogbf(mx) : 0;
    if (lane == 0) sigma_l[t * 4 + Sx] = sigma;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t q0, q1, q2;
      split3x4(ldexpf(v[i].x, sigma), ldexpf(v[i].y, sigma), ldexpf(v[i].z, sigma), ldexpf(v[i].w, sigma), q0, q1, q2);
      const uint32_t col = (Sx * 4 + i) * kXqChunk + 4 * lane;
      *reinterpret_cast<uint32_t*>(xq + (t * 3 + 0) * kXqRow + col) = q0;
      *reinterpret_cast<uint32_t*>(xq + (t * 3 + 1) * kXqRow + col) = q1;
      *reinterpret_cast<uint32_t*>(xq + (t * 3 + 2) * kXqRow + col) = q2;
    }
  };
  if constexpr (XF == kXDimMajor) {
    if (wv < xquads * nst) {
      // unit: token 4 g4 + c is component c of the row pieces; its columns 4 lane .. 4 lane + 3
      // of chunk i are rows r = 0..3 of xr[4 i + r]
      const uint32_t g4 = wv / nst, Sx = wv % nst;
      auto comp = [](float4 a, int c) { return c == 0 ? a.x : c == 1 ? a.y : c == 2 ? a.z : a.w; };
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (4 * g4 + c < M) {
          float4 v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            v[i] = make_float4(comp(xr[4 * i], c), comp(xr[4 * i + 1], c), comp(xr[4 * i + 2], c), comp(xr[4 * i + 3], c));
          stage_pair(4 * g4 + c, Sx, v[0], v[1], v[2], v[3]);
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const uint32_t p = wv + (uint32_t)j * kFW;
      if (p < M * nst) stage_pair(p / nst, p % nst, xr[4 * j], xr[4 * j + 1], xr[4 * j + 2], xr[4 * j + 3]);
    }
  }
  AFFX_TRACE(15);
  AFFX_TRACEW(0);
  build_lut<KC, kFT, 3, ROT>(lut_s, cbv, tid);
  if (tid < 64) reinterpret_cast<uint32_t*>(zero_l)[tid] = 0u;
  AFFX_TRACEW(1);
  if constexpr (SINGLE) {
    // Batch 1: a wave counts its share in, then issues its gate/up weight loads, then waits for
    // every wave's share. With the loads issued first and a workgroup barrier here, the barrier
    // waited for the waves still issuing loads (the third wave of each SIMD issues its loads about
    // 3 us after the first, held by the memory pipeline), and no wave could start on weights that
    // had arrived. Every wave counts in exactly once, before it waits, so the wait always ends
    // (the waves of a workgroup are resident together). The release add orders the wave's LDS
    // writes before its count; the acquire load and fence order the reads of the other waves'
    // writes after it. (Larger batches issue their loads first and keep the barrier: measured
    // faster there, where each wave's share of the activation split is three times larger.)
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) __hip_atomic_fetch_add(parts_in, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    load_gu(rounds > 0 ? gu_item(0) : ~0u);
    if (lane == 0)
      while (__hip_atomic_load(parts_in, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)kFW)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  } else {
    __syncthreads();  // plan, activation terms and codebook copies visible
    ns = __builtin_amdgcn_readfirstlane(parts_in[1]);
    set_counts();
    has_down = g < dtiles && wv < NU;
    plan_in_lds = true;
  }
  AFFX_TRACE(1);

  // B source of this lane for gate/up: its (token, term) row at this wave's segment
  const uint32_t c = lane & 15, kg = lane >> 4;
  const uint8_t* bsrc[CG];

  // ---- 4. gate/up rounds -----------------------------------------------------------------------
  const uint32_t n_rounds = SINGLE ? (rounds > 0 ? 1u : 0u) : rounds;
  for (uint32_t rho = 0; rho < n_rounds; ++rho) {
    const uint32_t item = gu_item(rho);
    v4f acc[2][CG];
    // this lane's token in each column group, and whether the lane writes that token's partial
    // sums (lanes of the first term column of a token)
    uint32_t tk[CG];
    bool tw[CG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      tk[cg] = 0u;
      tw[cg] = false;
    }
    // partial sums of this wave's segment, term-combined, at the segment's exponent:
    // part[wave][mat][row][token]. Accumulator lane l, element v = D[4(l/16)+v][l%16].
    auto write_part = [&]() {
#pragma unroll
      for (int mm = 0; mm < 2; ++mm)
#pragma unroll
        for (int cg = 0; cg < CG; ++cg)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float val = fused_terms(acc[mm][cg][v]);
            if (tw[cg]) part[((wv * 2 + mm) * 16 + 4 * kg + v) * M + tk[cg]] = ldexpf(val, -sigma_l[tk[cg] * 4 + S]);
          }
    };
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) acc[mm][cg] = v4f{0.f, 0.f, 0.f, 0.f};
    // (rounds kernels) this round's row scales, kept apart: the ring requests the next round's into
    // rs_gu during the steps (row scales are requested first, so the wait for them at their use
    // covers no weights)
    const uint32_t rs_cur = rs_gu;
    // Rounds kernels: the previous round's epilogue reads the partial sums and row scales in LDS
    // that this round rewrites. Instead of a workgroup barrier after that epilogue (every wave
    // idle for it), each wave counts itself in when its share of it is done, and a wave waits for
    // all of them only where it first writes those arrays: almost always long done by then.
    auto wait_epilogue = [&]() {
      if (!SINGLE && rho > 0) {
        if (lane == 0)
          while (__hip_atomic_load(parts_in + 2, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)kFW * rho)
            __builtin_amdgcn_s_sleep(1);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      }
    };
    if (item != ~0u) {
      const uint32_t slot = item / rt_per;
      const uint32_t mask = __builtin_amdgcn_readfirstlane(slot_mask[slot]);
      const uint32_t nt = (uint32_t)__builtin_popcount(mask);
      const uint32_t tl = CMP ? __builtin_amdgcn_readfirstlane(slot_tok[slot]) : 0u;
      const uint32_t npass = CMP ? (nt + 4u) / 5u : 1u;
      // the ring's part after step m of the last pass (unconditional: an absent next item reads
      // expert 0's first tile, never used, and straight-line loads keep the compiler's wait counts
      // exact). Step m + 1's table reads, issued before it, were the last reads of the registers
      // each part overwrites: chunk 0 after step 1's, chunk 1 after step 3's, chunk 2 after step
      // 4's, chunk 3 after step 6's, chunk 4 and the three field dwords (the last read by step 7's)
      // after step 7's.
      const uint32_t nit = RING ? gu_item(rho + 1) : ~0u;
      const bool nok = nit != ~0u;
      const uint32_t nrt = nok ? nit % rt_per : 0u;
      const uint8_t* nex = A.base + (uint64_t)(nok ? slot_expert_of(nit / rt_per) : 0u) * A.stride;
      const uint64_t ntile = nok ? (uint64_t)nrt * nst + S : 0u;
      const uint8_t* ngc = nex + A.off[kGateCodes] + ntile * kTileCodeBytes + lane * 16;
      const uint8_t* nuc = nex + A.off[kUpCodes] + ntile * kTileCodeBytes + lane * 16;
      const uint32_t* ngf = reinterpret_cast<const uint32_t*>(nex + A.off[kGateFields] + ntile * kTileFieldBytes + lane * 12);
      const uint32_t* nuf = reinterpret_cast<const uint32_t*>(nex + A.off[kUpFields] + ntile * kTileFieldBytes + lane * 12);
      auto ring = [&](int m) {
        auto chunk = [&](int j) {
          const u32x4 x0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ngc + j * 1024));
          const u32x4 x1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(nuc + j * 1024));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            ug.c[4 * j + i] = x0[i];
            uu.c[4 * j + i] = x1[i];
          }
        };
        auto fields = [&]() {  // (one 12-byte load each: fewer requests for the address unit)
          const u32x3a gv = __builtin_nontemporal_load(reinterpret_cast<const u32x3a*>(ngf));
          const u32x3a uv = __builtin_nontemporal_load(reinterpret_cast<const u32x3a*>(nuf));
#pragma unroll
          for (int i = 0; i < 3; ++i) {
            ug.f[i] = gv[i];
            uu.f[i] = uv[i];
          }
        };
        if (m == 0) {
          rs_gu = reinterpret_cast<const uint16_t*>(nex + A.off[lane < 16 ? kGateRs : kUpRs])[nrt * 16 + (lane & 15)];
          chunk(0);
        } else if (m == 2) {
          chunk(1);
        } else if (m == 3) {
          chunk(2);
        } else if (m == 5) {
          chunk(3);
        } else if (m == 6) {
          chunk(4);
          fields();
        }
      };
      // one pass over the weight registers per group of five of the slot's tokens; the ring runs in
      // the last pass only (an earlier pass must leave the registers as they are)
      auto gu_pass = [&](uint32_t p, auto ringc) {
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
          uint32_t t;
          bool valid;
          if constexpr (CMP) {
            valid = cmp_column(tl, nt, p, c, t);
          } else {
            t = cg * 5 + c / 3;
            valid = c < 15 && t < M && ((mask >> t) & 1u);
          }
          const uint32_t tau = c % 3;
          bsrc[cg] = valid ? xq + (t * 3 + tau) * kXqRow + (S * 4 + kg) * kXqChunk : zero_l;
          tk[cg] = t;
          tw[cg] = tau == 0 && (CMP ? valid : (c < 15 && t < M));
        }
        uint32_t rg[8], ru[8];
        uint32_t bg[2], bu[2];
        pin_step(ug, 0);
        pin_step(uu, 0);
        lut_lookup_step<KC, ROT>(ug, lut, btbl, copy4, 0, rg, bg);
        lut_lookup_step<KC, ROT>(uu, lut, btbl, copy4, 0, ru, bu);
        v8i bc[CG];
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) bc[cg] = b_step_lds(bsrc[cg], 0);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          // Issue priority falls with the step (3 for steps 0-1 down to 0 for steps 6-7): a wave
          // behind the others of its SIMD is issued first, so the three finish their steps closer
          // together. By age alone the oldest finished some 3 us before the youngest, which then
          // ran alone on the SIMD until the barrier (C3 1.0 %, C5 1.3 % faster measured).
          switch (m / 2) {
            case 0: __builtin_amdgcn_s_setprio(3); break;
            case 1: __builtin_amdgcn_s_setprio(2); break;
            case 2: __builtin_amdgcn_s_setprio(1); break;
            default: __builtin_amdgcn_s_setprio(0); break;
          }
          uint32_t ng[8], nu[8];
          uint32_t nbg[2], nbu[2];
          v8i bn[CG];
          if (m < 7) {
#pragma unroll
            for (int cg = 0; cg < CG; ++cg) { AFFX_PIN(acc[0][cg]); AFFX_PIN(acc[1][cg]); }
            pin_step(ug, m + 1);
            pin_step(uu, m + 1);
            lut_lookup_step<KC, ROT>(ug, lut, btbl, copy4, m + 1, ng, nbg);
            lut_lookup_step<KC, ROT>(uu, lut, btbl, copy4, m + 1, nu, nbu);
#pragma unroll
            for (int cg = 0; cg < CG; ++cg) bn[cg] = b_step_lds(bsrc[cg], m + 1);
          }
          const v8i ag = lut_finish(rg, bg), au = lut_finish(ru, bu);
#pragma unroll
          for (int cg = 0; cg < CG; ++cg) {
            acc[0][cg] = mfma(ag, bc[cg], acc[0][cg]);
            acc[1][cg] = mfma(au, bc[cg], acc[1][cg]);
          }
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (decltype(ringc)::value) {
            ring(m);
            __builtin_amdgcn_sched_barrier(0);
          }
          if (m < 7) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { rg[i] = ng[i]; ru[i] = nu[i]; }
            bg[0] = nbg[0]; bg[1] = nbg[1]; bu[0] = nbu[0]; bu[1] = nbu[1];
#pragma unroll
            for (int cg = 0; cg < CG; ++cg) bc[cg] = bn[cg];
          }
        }
      };
      if constexpr (CMP) {
        if (npass > 1) {
          gu_pass(0u, std::false_type{});
          wait_epilogue();
          write_part();  // (a slot with more than five tokens) the first pass's tokens are done
#pragma unroll
          for (int mm = 0; mm < 2; ++mm) acc[mm][0] = v4f{0.f, 0.f, 0.f, 0.f};
        }
      }
      gu_pass(npass - 1u, std::integral_constant<bool, RING>{});
    }
    AFFX_TRACE(3);
    if (!RING && item != ~0u && S == 0 && lane < 32) {
      // opaque at the use: no conversion is hoisted next to the load (its wait would then cover
      // every weight load issued before it)
      uint32_t rv = rs_gu;
      AFFX_PIN(rv);
      rs_l[q * 32 + lane] = __uint_as_float(rv << 16);
    }
    // one pass: a wave that stores no SwiGLU output issues its down unit now (its gate/up data is
    // in), so that it has arrived when the wave decodes it during the publish and wait. After the
    // row-scale write above: where a branch that issues loads joins, the compiler's wait for a
    // value loaded before the branch covers every load in flight, so the write would wait for
    // this unit (about 1 us).
    if constexpr (SINGLE && PREF) {
      if (wv >= epi_waves) load_down(has_down, g, wv);
    }
    wait_epilogue();
    if (RING && item != ~0u && S == 0 && lane < 32) rs_l[q * 32 + lane] = __uint_as_float(rs_cur << 16);
    write_part();  // (the last pass's tokens)
    __syncthreads();
    AFFX_TRACE(11);

    // epilogue: thread (group, row, token) sums the group's segments in order, SwiGLU, E4M3 terms
    // (up to 12 groups x 16 rows x 8 tokens: two passes of the workgroup)
    uint32_t et0 = tid;
    AFFX_PIN(et0);  // epilogue index math stays after the compute (no live range across it)
    // (a loop header here would make every wave with loads in flight wait for all of them, the
    // down prefetch included: SINGLE, with at most 12 x 16 threads busy, takes one pass)
    auto epilogue = [&](uint32_t et) {
      // (row fastest: the stores of 16 neighbouring lanes form one 16-byte run per term)
      const uint32_t qq = et / (16 * M), t = (et / 16) % M, r = et % 16;
      const uint32_t k = rho * groups + qq;
      if (k < my_items) {
        const uint32_t it = g + A.n_wg * k, slot = it / rt_per, rt = it % rt_per;
        if ((slot_mask[slot] >> t) & 1u) {
          float s2[2];
#pragma unroll
          for (int mm = 0; mm < 2; ++mm) {
            float sum = 0.f;
            for (uint32_t sg = 0; sg < nst; ++sg) sum += part[(((qq * nst + sg) * 2 + mm) * 16 + r) * M + t];
            s2[mm] = sum;
          }
          const uint32_t row = rt * 16 + r;
          float gg = s2[0] * rs_l[qq * 32 + r], uu2 = s2[1] * rs_l[qq * 32 + 16 + r];
          // SwiGLU with the asymmetric clamp: src/engine/ops.cpp:47-60
          const float Lm = A.limit;
          gg = (Lm < gg) ? Lm : gg;
          const float lo = (-Lm < uu2) ? uu2 : -Lm;
          uu2 = (lo < Lm) ? lo : Lm;
          const float a = (gg / (1.0f + expf(-gg))) * uu2;
          uint32_t b0, b1, b2;
          split3(ldexpf(a, A.sigma_a), b0, b1, b2);
          // device-coherent stores (written through to the memory side before they complete)
          uint8_t* dst = A.aq + ((uint64_t)(slot * M + t) * kTerms) * A.inter + row;
          __hip_atomic_store(dst, (uint8_t)b0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(dst + A.inter, (uint8_t)b1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(dst + 2 * (uint64_t)A.inter, (uint8_t)b2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    };
    if constexpr (SINGLE) {
      if (et0 < groups * 16 * M) epilogue(et0);
    } else {
      for (uint32_t et = et0; et < groups * 16 * M; et += kFT) epilogue(et);
    }
    if constexpr (!SINGLE) {
      // this wave's reads of the round's partial sums and row scales are done (release: ordered
      // before the next round's writes of the other waves, which acquire the count)
      __builtin_amdgcn_wave_barrier();
      if (lane == 0) __hip_atomic_fetch_add(parts_in + 2, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }

  // The first down unit's weights are loaded now, after this workgroup's gate/up data has arrived
  // (issued earlier they would share the HBM stream with it and delay gate/up), so they stream in
  // while the layer publishes and waits.
  //
  // Publish (once, all rounds). Why the SwiGLU output is visible to every down workgroup, on any
  // XCD, without a release fence (the memory-model argument; a formal agent-scope release here
  // measured 2.7 to 8.4 us per layer slower: its L2 write-back, and its wait for the down-unit
  // loads in flight in the releasing wave):
  //  * every value handed across is written by an agent-scope atomic store, which the compiler
  //    emits as `global_store ... sc1`; its own mapping of agent-scope atomics treats such a store
  //    as visible to the whole device once it has completed (it emits no L2 write-back for it:
  //    the write-back of a release is for non-atomic stores, and there are none to hand over);
  //  * each storing wave waits for its stores to complete: vector memory operations complete in
  //    issue order (the property the compiler's own waits rely on when they wait for one load
  //    among several with vmcnt(N) > 0), and only the nine loads of the down unit were issued
  //    after the stores, so vmcnt(7) covers them;
  //  * the barrier orders those waits before thread 0's counter add; the add that completes the
  //    count is performed after every other add, hence after every workgroup's stores completed;
  //    its wave reads the old value back before it raises the flags, so the add is performed
  //    before any flag store is issued;
  //  * rounds kernels: a waiter that sees its flag runs an agent-scope acquire fence
  //    (`buffer_inv sc1`) before any workgroup thread reads the SwiGLU output, so no stale line of
  //    an earlier launch is read from its CU's or its XCD's caches;
  //  * the one-pass kernel instead reads the SwiGLU output with loads that carry the same
  //    device-coherence bit (`buffer_load ... sc1`, what the compiler emits for an agent-scope
  //    atomic load), issued only after the publish flags were seen (a compiler barrier after the
  //    poll, the workgroup barrier for the other waves): such a load reads past the non-coherent
  //    caches, so it needs no invalidate. The acquire's L2 invalidate, once per workgroup, had
  //    every workgroup of an XCD refetch the others' lines: 19.8 against 18.3 us per layer.
  if (!SINGLE || n_rounds == 0 || wv < epi_waves) load_down(has_down, g, wv);
  if (n_rounds > 0 && wv < epi_waves) __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(7));
  AFFX_TRACE(10);
  __syncthreads();
  // Batch 1 (one pass): no counter. Every workgroup, items or not, publishes epoch + 1 in its own
  // dword of each replica of the publish flags once its stores have completed (the barrier above
  // orders the storing waves' waits before these stores). A waiter polls one replica and is
  // released when every workgroup of the launch has published: one round trip less than the
  // counter add and the flag fan-out that follows it.
  uint32_t ep = 0;
  if constexpr (SINGLE) {
    uint32_t er = ep_raw;
    AFFX_PIN(er);  // the epoch's wait stays here
    ep = __builtin_amdgcn_readfirstlane(er) + 1u;
    if (wv == 0 && lane < kPubReplicas)
      __hip_atomic_store(A.sync + (kPubOff + lane * kPubStride) / 4 + g, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!SINGLE && wv == 0 && n_rounds > 0) {
    // the add that completes the count clears it for the next launch and raises the flag of each
    // waiting workgroup (one line each: the waiters poll without contending for one address)
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(&A.sync[0], my_items, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readlane(old, 0);
    if (old + my_items == NI) {
      if (lane == 0) __hip_atomic_store(&A.sync[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t nwait = A.n_wg < dtiles ? A.n_wg : dtiles;
      for (uint32_t i = lane; i < nwait; i += 64)
        __hip_atomic_store(A.sync + (kSyncHeader + i * kSyncFlagStride) / 4, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  AFFX_TRACE(4);
  // ---- 4b. one pass (batch 1): the A fragments of this wave's first down unit (the one loaded
  // before the publish) do not depend on the activations, so all eight steps are decoded now,
  // while the layer publishes and this workgroup waits; after the release only the staging of
  // the activations and eight MFMAs remain for it

  constexpr int kPreSteps = 8;
  v8i ad[SINGLE ? kPreSteps : 1];
  if constexpr (SINGLE) {
    if (has_down) {
#pragma unroll
      for (int m = 0; m < kPreSteps; ++m) {
        uint32_t raw[8], bv[2];
        pin_step(ud, m);
        lut_lookup_step<KC, ROT>(ud, lut, btbl, copy4, m, raw, bv);
        ad[m] = lut_finish(raw, bv);
      }
    }
  }
  AFFX_TRACE(14);
  // ---- 5. wait for every gate/up item (this workgroup's flag), then the down tiles -------------
  if (g < dtiles) {
    if (SINGLE && wv == 0 && NI > 0) {
      // every workgroup's publish flag in this workgroup's replica, four per lane
      const __amdgpu_buffer_rsrc_t fr =
          buffer_rsrc(reinterpret_cast<const uint8_t*>(A.sync) + kPubOff + (g % kPubReplicas) * kPubStride, kPubStride);
      for (uint32_t n = 0;; ++n) {
        if (n >= A.spin_limit) {
          if (lane == 0)
            __hip_atomic_fetch_or(&A.sync[kSyncErrWord], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        const u32x4 f = __builtin_amdgcn_raw_buffer_load_b128(fr, 16u * lane, 0, kDevCoherent);
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) ok = ok && (4u * lane + i >= A.n_wg || f[i] == ep);
        if (__ballot(!ok) == 0ull) break;
        __builtin_amdgcn_s_sleep(2);
        asm volatile("" ::: "memory");  // the next poll reloads
      }
      // every workgroup has read the epoch (each published epoch + 1): the next launch's epoch
      if (g == 0 && lane == 0) __hip_atomic_store(&A.sync[kEpochWord], ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // (no acquire fence: the SwiGLU output is read with device-coherent loads, see the publish;
      // the compiler may not move those loads above this point)
      asm volatile("" ::: "memory");
    }
    if (!SINGLE && tid == 0 && NI > 0) {
      uint32_t* flag = A.sync + (kSyncHeader + g * kSyncFlagStride) / 4;
      // at most spin_limit polls (none at 0: the give-up path runs deterministically)
      for (uint32_t n = 0;; ++n) {
        if (n >= A.spin_limit) {
          __hip_atomic_fetch_or(&A.sync[kSyncErrWord], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
        __builtin_amdgcn_s_sleep(2);
      }
      __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next launch
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    AFFX_TRACE(5);

    const uint32_t rg4 = lane >> 4;
    // one output tile; PRE: its first unit per wave was decoded before the wait (a separate
    // instantiation, so that those fragments are not live across the loop over further tiles)
    auto down_tile = [&](uint32_t td, auto prec) {
      constexpr bool PRE = decltype(prec)::value;
      // per (row, token) sums of this wave's units: in registers by column (the column's token is
      // fixed), or, with compacted columns (the token of a column changes from unit to unit),
      // added in place in this wave's rows of part[wave][row][token], in the same unit order
      float yacc[CG][4];
#pragma unroll
      for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int v = 0; v < 4; ++v) yacc[cg][v] = 0.f;
      if constexpr (CMP) {
        for (uint32_t i = lane; i < 16u * M; i += 64u) part[wv * 16u * M + i] = 0.f;
      }
#pragma unroll 1
      for (uint32_t u = wv; u < (SINGLE ? (wv < NU ? wv + 1 : 0u) : NU); u += kFW) {
        if (!(PRE || (PREF && td == g && u == wv))) load_down(true, td, u);  // else loaded before the wait
        const uint32_t slot = u / nsi, S2 = u % nsi;
        const uint32_t mask = __builtin_amdgcn_readfirstlane(slot_mask[slot]);
        uint2 rsv = rs_d;
        AFFX_PIN(rsv.x);  // opaque at the use (see the gate/up row scales)
        AFFX_PIN(rsv.y);
        const uint32_t nt = (uint32_t)__builtin_popcount(mask);
        const uint32_t tl = CMP ? __builtin_amdgcn_readfirstlane(slot_tok[slot]) : 0u;
        const uint32_t npass = CMP ? (nt + 4u) / 5u : 1u;
        for (uint32_t p = 0; p < npass; ++p) {
          BSrc<CG> b;
          uint32_t tcol = 0;  // (compacted columns) this lane's token
          if constexpr (CMP) {
            b.used = cmp_column(tl, nt, p, c, tcol);
            b.p[0] = b.used ? reinterpret_cast<const u32x4*>(A.aq + ((uint64_t)(slot * M + tcol) * kTerms + c % 3) * A.inter +
                                                             (uint64_t)S2 * kTileCols + kg * kSegCols)
                            : reinterpret_cast<const u32x4*>(A.zeros);
          } else {
            b = b_source<CG>(A.aq + (uint64_t)slot * M * kTerms * A.inter, A.inter, (uint64_t)S2 * kTileCols, lane, M,
                             mask, A.zeros);
          }
          __builtin_amdgcn_sched_barrier(0);
          v4f acc[CG];
#pragma unroll
          for (int cg = 0; cg < CG; ++cg) acc[cg] = v4f{0.f, 0.f, 0.f, 0.f};
          // B: the column group (64 registers) is loaded whole up front, so the eight steps wait
          // for one round trip; only the lanes of used columns load (exec-masked), the others hold
          // zeros, with no address-unit time spent on a zero run
          v8i bpre[8];
#pragma unroll
          for (int m = 0; m < 8; ++m) bpre[m] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
          if (b.used) {
#pragma unroll
            for (int m = 0; m < 8; ++m) bpre[m] = b_step(b.p[0], m);
          }
          __builtin_amdgcn_sched_barrier(0);
          // steps [m0, 8) decode their A fragments here (PRE: the first kPreSteps are in ad)
          constexpr int m0 = PRE ? kPreSteps : 0;
          if constexpr (PRE) {
#pragma unroll
            for (int m = 0; m < m0; ++m) acc[0] = mfma(ad[SINGLE ? m : 0], bpre[m], acc[0]);
          }
          {
            uint32_t raw[8];
            uint32_t bv[2];
            pin_step(ud, m0);
            lut_lookup_step<KC, ROT>(ud, lut, btbl, copy4, m0, raw, bv);
#pragma unroll
            for (int m = m0; m < 8; ++m) {
              uint32_t nraw[8];
              uint32_t nbv[2];
              if (m < 7) {
                // the previous step's MFMA stays ahead of these reads (else the compiler sinks every
                // MFMA below all eight steps' table reads and holds them all in registers)
#pragma unroll
                for (int cg = 0; cg < CG; ++cg) AFFX_PIN(acc[cg]);
                pin_step(ud, m + 1);
                lut_lookup_step<KC, ROT>(ud, lut, btbl, copy4, m + 1, nraw, nbv);
              }
              acc[0] = mfma(lut_finish(raw, bv), bpre[m], acc[0]);
              __builtin_amdgcn_sched_barrier(0);
              if (m < 7) {
#pragma unroll
                for (int i = 0; i < 8; ++i) raw[i] = nraw[i];
                bv[0] = nbv[0]; bv[1] = nbv[1];
              }
            }
          }
          const float rs[4] = {__uint_as_float(rsv.x << 16), __uint_as_float(rsv.x & 0xFFFF0000u),
                               __uint_as_float(rsv.y << 16), __uint_as_float(rsv.y & 0xFFFF0000u)};
#pragma unroll
          for (int cg = 0; cg < CG; ++cg) {
            const uint32_t t = CMP ? tcol : cg * 5 + c / 3;
            const bool mine = CMP ? b.used && (c % 3) == 0 : c < 15 && (c % 3) == 0 && t < M && ((mask >> t) & 1u);
            const float wt = mine ? ldexpf(slot_w[slot * M + t], -A.sigma_a) : 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const float val = fused_terms(acc[cg][v]);
              if (mine) {
                if constexpr (CMP) part[(wv * 16 + 4 * rg4 + v) * M + t] += val * rs[v] * wt;
                else yacc[cg][v] += val * rs[v] * wt;
              }
            }
          }
        }
      }
      AFFX_TRACE(6);
      // per-wave partials [wave][row][token], summed over the waves in order
      if constexpr (!CMP) {
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
          const uint32_t t = cg * 5 + c / 3;
          if (c < 15 && c % 3 == 0 && t < M)
#pragma unroll
            for (int v = 0; v < 4; ++v) part[(wv * 16 + 4 * rg4 + v) * M + t] = yacc[cg][v];
        }
      }
      __syncthreads();
      uint32_t et = tid;
      AFFX_PIN(et);
      if (et < 16 * M) {
        const uint32_t r = et / M, t = et % M;
        float sum = 0.f;
        for (int qw = 0; qw < kFW; ++qw) sum += part[(qw * 16 + r) * M + t];
        float* dst = A.y + (uint64_t)t * A.yts + (uint64_t)(td * 16 + r) * A.yds;
        *dst = A.accumulate ? *dst + sum : sum;
      }
      __syncthreads();
    };
    uint32_t td0 = g;
    if constexpr (SINGLE) {
      // Batch 1, the first output tile, its eight down steps already decoded (ad). When every
      // workgroup has one output tile (the grid covers the hidden rows: the device-filling case),
      // the SwiGLU terms of all units (at most 12 units x 3 terms x 1024 columns = 36 KiB,
      // [slot][term][inter] as in memory) are copied into LDS over the codebook tables, which
      // the barrier above frees: one coalesced 16-byte device-coherent load per thread and round
      // (see the publish) instead of each wave's scattered 256-byte runs; each wave then reads
      // its B operand from LDS (only the lanes of used columns). A workgroup with further tiles
      // keeps the tables for them and reads its first tile's operand from memory as they do
      // (plain loads after the acquire fence).
      const bool staged = A.n_wg >= dtiles;
      static_assert(Lut<KC, ROT>::kDwords * 4 >= (int)(kPollUnitsMax * kTerms * kTileCols), "staging fits the tables");
      if (staged) {
        const uint32_t n16 = ns * kTerms * A.inter / 16u;
        u32x4* dst = reinterpret_cast<u32x4*>(lut_s);
        const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(A.aq, n16 * 16u);
        for (uint32_t i = tid; i < n16; i += kFT)
          dst[i] = __builtin_amdgcn_raw_buffer_load_b128(ar, 16u * i, 0, kDevCoherent);
      } else {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
      __syncthreads();
      {
        float yacc[4] = {0.f, 0.f, 0.f, 0.f};
        if (has_down) {
          const uint32_t slot = wv / nsi, S2 = wv % nsi;
          const uint32_t mask = __builtin_amdgcn_readfirstlane(slot_mask[slot]);
          const bool used = c < 3u && (mask & 1u) != 0u;
          const uint64_t boff = (uint64_t)(slot * kTerms + (used ? c : 0u)) * A.inter + S2 * kTileCols + kg * kSegCols;
          const uint8_t* bl = reinterpret_cast<const uint8_t*>(lut_s) + boff;
          const u32x4* bg = reinterpret_cast<const u32x4*>(A.aq + boff);
          uint2 rsv = rs_d;
          AFFX_PIN(rsv.x);
          AFFX_PIN(rsv.y);
          v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int m = 0; m < 8; ++m) {
            v8i b = v8i{0, 0, 0, 0, 0, 0, 0, 0};
            if (used) b = staged ? b_step_lds(bl, m) : b_step(bg, m);
            acc = mfma(ad[m], b, acc);
          }
          const float rs[4] = {__uint_as_float(rsv.x << 16), __uint_as_float(rsv.x & 0xFFFF0000u),
                               __uint_as_float(rsv.y << 16), __uint_as_float(rsv.y & 0xFFFF0000u)};
          const bool mine = c == 0u && (mask & 1u) != 0u;
          const float wt = mine ? ldexpf(slot_w[slot * M], -A.sigma_a) : 0.f;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float val = fused_terms(acc[v]);
            if (mine) yacc[v] += val * rs[v] * wt;
          }
        }
        AFFX_TRACE(6);
        if (c == 0u) {
#pragma unroll
          for (int v = 0; v < 4; ++v) part[wv * 16 + 4 * rg4 + v] = yacc[v];
        }
        __syncthreads();
        uint32_t et = tid;
        AFFX_PIN(et);
        if (et < 16u) {
          float sum = 0.f;
          for (int qw = 0; qw < kFW; ++qw) sum += part[qw * 16 + et];
          float* dst = A.y + (uint64_t)(g * 16 + et) * A.yds;
          *dst = A.accumulate ? *dst + sum : sum;
        }
        __syncthreads();  // (this tile's partial sums read before the next tile rewrites them)
      }
      td0 += A.n_wg;
    }
    for (uint32_t td = td0; td < dtiles; td += A.n_wg) down_tile(td, std::false_type{});
  }

  AFFX_TRACE(7);
}

}  // namespace affx

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
using namespace affx;

namespace {

struct FusedVariant {
  const void* fn;
  void (*launch)(uint32_t n_wg, uint32_t lds, hipStream_t st, const FusedArgs& A);
  uint32_t kc, maxm;
  int max_wg;  // workgroups the device holds at once (0: cannot run)
  bool ready;
};

template <int CG, int KC, int MAXM, bool SINGLE, int XF>
void launch_fused(uint32_t n_wg, uint32_t lds, hipStream_t st, const FusedArgs& A) {
  hipLaunchKernelGGL((decode_fused_kernel<CG, KC, MAXM, SINGLE, true, XF>), dim3(n_wg), dim3(kFT), lds, st, A);
}

template <int CG, int KC, int MAXM, bool SINGLE, int XF>
FusedVariant fused_entry() {
  FusedVariant f{};
  f.fn = (const void*)decode_fused_kernel<CG, KC, MAXM, SINGLE, true, XF>;
  f.launch = launch_fused<CG, KC, MAXM, SINGLE, XF>;
  f.kc = KC;
  f.maxm = MAXM;
  return f;
}

constexpr int kMaxDev = 64;
std::mutex g_fused_mu;
FusedVariant g_fused[kMaxDev][4][3];

// variants (all with the rotated tables): 0 M = 1 in one pass (8 codebook copies), 1 M = 1 in
// rounds, 2 M <= 5 (4 copies), 3 M <= 8 (2 copies, compacted columns). The larger M, the more LDS
// the activation terms take; the copies fill what is left.
int fused_variant(uint32_t M, bool single) { return M == 1 ? (single ? 0 : 1) : M <= 5 ? 2 : 3; }

// Polls of a release flag before a waiter gives up: kSpinLimit, or AFFX_DECODE_SPIN_LIMIT from
// the environment (read at every call; a test makes the wait give up with a small value, so the
// failure path runs with every kernel still exiting normally).
uint32_t decode_spin_limit() {
  const char* e = getenv("AFFX_DECODE_SPIN_LIMIT");
  return e && *e ? (uint32_t)strtoul(e, nullptr, 10) : kSpinLimit;
}

// the XForm for these strides
int fused_xform(const float* x, uint64_t x_ts, uint64_t x_ds, uint32_t M, uint32_t hidden) {
  const bool al = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  if (x_ds == 1 && (M == 1 || (x_ts & 3u) == 0) && al) return kXTokenMajor;
  const uint32_t quads = (M + 3) / 4, nst = hidden / kTileCols;
  if (x_ts == 1 && (x_ds & 3u) == 0 && x_ds >= 4u * quads && al && quads * nst <= (uint32_t)kFW)
    return kXDimMajor;
  return kXStrided;
}

int fused_prepare(int dev, int v, int xf, FusedVariant* out) {
  std::lock_guard<std::mutex> lk(g_fused_mu);
  FusedVariant& f = g_fused[dev][v][xf];
  if (!f.ready) {
    static const FusedVariant table[4][3] = {
        {fused_entry<1, 8, 1, true, kXStrided>(), fused_entry<1, 8, 1, true, kXTokenMajor>(),
         fused_entry<1, 8, 1, true, kXDimMajor>()},
        {fused_entry<1, 8, 1, false, kXStrided>(), fused_entry<1, 8, 1, false, kXTokenMajor>(),
         fused_entry<1, 8, 1, false, kXDimMajor>()},
        {fused_entry<1, 4, 5, false, kXStrided>(), fused_entry<1, 4, 5, false, kXTokenMajor>(),
         fused_entry<1, 4, 5, false, kXDimMajor>()},
        {fused_entry<1, 2, 8, false, kXStrided>(), fused_entry<1, 2, 8, false, kXTokenMajor>(),
         fused_entry<1, 2, 8, false, kXDimMajor>()}};
    if (!table[v][xf].fn) return set_error(AFFX_ERR_ARG, "ffn_decode: no fused kernel for variant %d form %d", v, xf);
    f = table[v][xf];
    const uint32_t lds = fused_lds(f.maxm).total;  // dynamic part (the codebook copies are static)
    int rc = check_hip(hipFuncSetAttribute(f.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                       "hipFuncSetAttribute(fused decode)");
    if (rc) return rc;
    int per_cu = 0, cus = 0;
    rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f.fn, kFT, lds),
                   "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (rc) return rc;
    rc = check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
                   "hipDeviceGetAttribute");
    if (rc) return rc;
    f.max_wg = per_cu * cus;
    f.ready = true;
  }
  *out = f;
  return AFFX_OK;
}

}  // namespace

extern "C" int affx_expert_ffn_decode(const affx_layer* L, const float* x, uint64_t x_ts,
                                      uint64_t x_ds, uint32_t M, const uint32_t* sel, const float* w,
                                      uint32_t K, float* y, uint64_t y_ts, uint64_t y_ds,
                                      int accumulate, void* ws, size_t ws_bytes, void* stream) {
  if (!x || !sel || !w || !y) return set_error(AFFX_ERR_ARG, "ffn_decode: null pointer");
  DecodeWs lay;
  int rc = decode_check(L, M, K, ws, ws_bytes, &lay);
  if (rc) return rc;
  if ((uint64_t)M * K > (uint64_t)kPlanRoutes)
    return set_error(AFFX_DECLINED, "ffn_decode: m_tokens * top_k must be <= %d", kPlanRoutes);
  int dev = 0;
  rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDev) return set_error(AFFX_ERR_ARG, "ffn_decode: device id %d", dev);
  const uint32_t nst = L->hidden / kTileCols, groups = kFW / nst;
  const uint32_t slots_max = M * K < L->n_experts ? M * K : L->n_experts;
  const uint32_t items_max = slots_max * (L->inter / kTileRows);
  const uint32_t dtiles = L->hidden / kTileRows;
  const uint32_t units_max = slots_max * (L->inter / kTileCols);
  uint32_t want = (items_max + groups - 1) / groups;
  if (want < dtiles) want = dtiles;
  FusedVariant f;
  const int xf = fused_xform(x, x_ts, x_ds, M, L->hidden);
  rc = fused_prepare(dev, fused_variant(M, false), xf, &f);  // any variant: the grid capacity
  if (rc) return rc;
  // the kernel addresses x with 32-bit element offsets; larger arenas take the staged launches
  const bool x_small = (uint64_t)M * x_ts + (uint64_t)L->hidden * x_ds < (1ull << 30);
  if (f.max_wg <= 0 || !x_small)
    return affx_decode_staged(L, x, x_ts, x_ds, M, sel, w, K, y, y_ts, y_ds, accumulate, ws, ws_bytes, stream);
  uint32_t n_wg = want < (uint32_t)f.max_wg ? want : (uint32_t)f.max_wg;
  // one pass: every gate/up item has its own wave group, every down unit of a tile its own wave
  bool single = items_max <= groups * n_wg && units_max <= (uint32_t)kFW;
  const int v = fused_variant(M, single);
  if (v != fused_variant(M, false)) {
    // the one-pass kernel is another instantiation: its own occupancy bounds the grid (every
    // workgroup must be resident at once), and a smaller grid may no longer hold every item in
    // one pass, in which case the rounds kernel runs on the grid that its own occupancy allows
    rc = fused_prepare(dev, v, xf, &f);
    if (rc) return rc;
    if (f.max_wg <= 0 || n_wg > (uint32_t)f.max_wg) {
      rc = fused_prepare(dev, fused_variant(M, false), xf, &f);
      if (rc) return rc;
      single = false;
    }
  }
  if (f.max_wg <= 0 || n_wg > (uint32_t)f.max_wg)
    return affx_decode_staged(L, x, x_ts, x_ds, M, sel, w, K, y, y_ts, y_ds, accumulate, ws, ws_bytes, stream);

  FusedArgs A;
  uint64_t off9[9];
  affx_expert_layout(L->hidden, L->inter, off9, nullptr);
  uint8_t* base = (uint8_t*)ws;
  A.base = (const uint8_t*)L->base;
  A.stride = L->stride;
  for (int i = 0; i < 9; ++i) A.off[i] = off9[i];
  A.hidden = L->hidden;
  A.inter = L->inter;
  A.M = M;
  A.K = K;
  A.n_experts = L->n_experts;
  A.n_wg = n_wg;
  A.codebook = (const uint32_t*)L->codebook;
  A.x = x;
  A.xts = x_ts;
  A.xds = x_ds;
  A.sel = sel;
  A.w = w;
  A.aq = base + lay.aq;
  A.zeros = base + lay.zeros;
  A.sync = (uint32_t*)(base + lay.sync);
  A.y = y;
  A.yts = y_ts;
  A.yds = y_ds;
  A.accumulate = accumulate;
  A.limit = L->swiglu_limit;
  A.sigma_a = 7 - ilogbf(L->swiglu_limit * L->swiglu_limit);
  A.spin_limit = decode_spin_limit();
  const uint32_t lds = fused_lds(M).total;
  hipStream_t st = (hipStream_t)stream;
  // the down B operand's unused columns read the workspace's zero run: zero in a zero-filled
  // workspace and only ever rewritten with zeros (by the staged prep kernel)
  f.launch(n_wg, lds, st, A);
  return check_launch("decode_fused_kernel");
}
