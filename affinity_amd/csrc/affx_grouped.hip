// Prefill path: the routed experts of a whole chunk, grouped by expert (each expert's weights
// are decoded once per tile of its tokens), on the fp8 MFMA.
//
//   grouped_plan     one workgroup: per-expert counts (from the routes, or from a slot list the
//                    caller built), exclusive scan, tile lists
//   grouped_run      per route: `run` (token t's routes are entries t k .. t k + k - 1 of `ord`)
//                    and a no-slot mark in `ord` for a route naming no expert of the layer
//   grouped_place    one workgroup per expert: its (token, route) pairs in token order (stable),
//                    so every slot and every output sum has a fixed order; writes the slot list
//                    (token and weight per slot, `ord`: each token's slots in route order)
//   grouped_prep_x   per token: exponent and E4M3 terms of the activation (2 terms for a bf16
//                    input: exact for every element of at least 2^-13 of the token's largest
//                    magnitude, where both terms are normal E4M3 numbers, and within 2^-20 of that
//                    maximum below it; 3 when a low bf16 term is given)
//   (each GEMM runs three times: the wide tiles, then the mid and the narrow ones, an expert's
//   partial last tile of at most kGMid or kGNarrow column tiles of tokens, in instantiations
//   whose MFMAs, fragment reads and direct loads cover just those columns)
//   grouped_gemm<0>  gate/up: (row block of 128 inter rows, token tile): 8 waves x 16 rows of
//                    gate and the same 16 of up, K = hidden in 128-column MFMA steps, 12 column
//                    tiles per A fragment; epilogue combines terms, applies row scales, SwiGLU,
//                    writes the activation as terms
//   grouped_gemm<1>  down: (row block of 256 hidden rows, slot tile): 8 waves x 32 rows, same
//                    structure over K = inter, writes each slot's unweighted down output z[slot]
//   grouped_combine  y[t] (+)= sum over token t's slots in `ord` order of wt[slot] * z[slot]
//
// Reference counterparts: run_batch_device's prefill arm (src/gpu/static_placement.hip:
// 1348-1964): moe_plan_kernel (src/gpu/moe_plan.hip:116-380), batch_quant_fp8_kernel
// (src/gpu/batch_kernels.hip:146-211), expert_gemm_wmma_kernel (src/gpu/expert_kernel.hip:
// 364-825), expert_swiglu_quant_kernel (862-931), expert_scatter_slots_kernel (935-947).
#include "affx_lut.h"

namespace affx {

constexpr int kPlanThreads = 1024;

struct Tile {
  uint32_t expert, slot0, n;
};

// Tiles of each GEMM by width class: wide (kGCT column tiles of tokens: every full tile, and a
// partial one that needs more than kGMid), mid (an expert's partial last tile of at most kGMid) and
// narrow (at most kGNarrow), stored in that order; each class runs in its own instantiation of the
// GEMM.
constexpr int kNCls = 3;
struct GroupedHdr {
  uint32_t n_slots;
  uint32_t tx;                     // activation terms of the gate/up input (2 or 3)
  uint32_t bad;                    // a caller's slot list needed more tiles than it can hold
  uint32_t n_cls[2][kNCls];        // [GEMM][class] tile counts
};

// ------------------------------------------------------------------------------------------------
// plan
// ------------------------------------------------------------------------------------------------
// Exclusive scan over the workgroup (kPlanThreads threads, thread i holds v[i]) of N counts at
// once; returns thread i's prefixes and writes the totals to tot.
template <int N>
__device__ __forceinline__ void plan_scan(uint32_t (&v)[N], uint32_t* wsum, uint32_t (&tot)[N]) {
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr uint32_t kW = kPlanThreads / 64;
  uint32_t inc[N];
#pragma unroll
  for (int q = 0; q < N; ++q) inc[q] = v[q];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1)
#pragma unroll
    for (int q = 0; q < N; ++q) {
      const uint32_t n = __shfl_up(inc[q], o);
      if (lane >= (uint32_t)o) inc[q] += n;
    }
  if (lane == 63)
#pragma unroll
    for (int q = 0; q < N; ++q) wsum[q * kW + wv] = inc[q];
  __syncthreads();
#pragma unroll
  for (int q = 0; q < N; ++q) {
    uint32_t before = 0, all = 0;
    for (uint32_t w = 0; w < kW; ++w) {
      const uint32_t x = wsum[q * kW + w];
      before += w < wv ? x : 0u;
      all += x;
    }
    v[q] = before + inc[q] - v[q];
    tot[q] = all;
  }
}

// Width class of an expert's partial last tile of r tokens (r > 0): 2 narrow, 1 mid, 0 wide; nar
// and mid are the token capacities of the narrow and mid widths.
__device__ __forceinline__ uint32_t tile_cls(uint32_t r, uint32_t nar, uint32_t mid) {
  return r <= nar ? 2u : r <= mid ? 1u : 0u;
}
// An expert's c slots in tiles of tt tokens: how many tiles of class k it has.
__device__ __forceinline__ uint32_t n_cls_of(uint32_t c, uint32_t tt, uint32_t nar, uint32_t mid, uint32_t k) {
  const uint32_t r = c % tt;
  return (k == 0 ? c / tt : 0u) + (r != 0u && tile_cls(r, nar, mid) == k ? 1u : 0u);
}
// Writes the tiles of one expert (slots b0 .. b0 + c - 1): the full ones from tiles[at[0]], the
// partial one at tiles[at[its class]] (at[0] past the full ones for a wide partial tile).
__device__ __forceinline__ void put_tiles(Tile* tiles, uint32_t e, uint32_t b0, uint32_t c, uint32_t tt, uint32_t nar,
                                          uint32_t mid, const uint32_t (&at)[kNCls]) {
  const uint32_t full = c / tt, r = c % tt;
  for (uint32_t k = 0; k < full; ++k) tiles[at[0] + k] = Tile{e, b0 + k * tt, tt};
  if (r > 0) {
    const uint32_t k = tile_cls(r, nar, mid);
    tiles[k == 0 ? at[0] + full : at[k]] = Tile{e, b0 + full * tt, r};
  }
}

// start_in: a caller's slot list, expert e owning slots [start_in[e], start_in[e+1]) of n_slots_in
// (each bound clamped to n_slots_in; a range that runs backwards is empty); null: count the routes.
__global__ void __launch_bounds__(kPlanThreads) grouped_plan_kernel(
    uint32_t* __restrict__ hist, uint32_t n_chunks, uint32_t n_experts, uint32_t tt1,
    uint32_t tt2, uint32_t nar1, uint32_t nar2, uint32_t mid1, uint32_t mid2, uint32_t tx,
    const uint32_t* __restrict__ start_in,
    uint32_t n_slots_in, uint32_t max_tiles1, uint32_t max_tiles2, GroupedHdr* __restrict__ hdr,
    uint32_t* __restrict__ offsets, Tile* __restrict__ tiles1, Tile* __restrict__ tiles2) {
  static_assert(AFFX_MAX_EXPERTS <= kPlanThreads, "one thread per expert in the scan");
  __shared__ uint32_t wsum[(1 + 2 * kNCls) * (kPlanThreads / 64)];
  const uint32_t tid = threadIdx.x;
  uint32_t c = 0, b0 = 0;
  if (start_in) {
    if (tid < n_experts) {
      const uint32_t a = min(start_in[tid], n_slots_in), b = min(start_in[tid + 1], n_slots_in);
      c = b > a ? b - a : 0u;
      b0 = a;
    }
  } else if (tid < n_experts) {
    // an expert's count: the sum of its chunk counts (grouped_hist_kernel), in chunk order
    for (uint32_t b = 0; b < n_chunks; ++b) c += hist[(uint64_t)b * n_experts + tid];
  }
  // slot offsets and tile offsets: one exclusive scan (expert order) of the count and the tiles of
  // each width class of both GEMMs
  constexpr int NV = 1 + 2 * kNCls;
  uint32_t v[NV], tot[NV];
  v[0] = c;
#pragma unroll
  for (int k = 0; k < kNCls; ++k) {
    v[1 + k] = n_cls_of(c, tt1, nar1, mid1, k);
    v[1 + kNCls + k] = n_cls_of(c, tt2, nar2, mid2, k);
  }
  plan_scan<NV>(v, wsum, tot);
  if (!start_in) b0 = v[0];
  uint32_t need1 = 0, need2 = 0;
#pragma unroll
  for (int k = 0; k < kNCls; ++k) { need1 += tot[1 + k]; need2 += tot[1 + kNCls + k]; }
  // a caller's overlapping ranges could ask for more tiles than the workspace holds: then no tile
  const bool fits = need1 <= max_tiles1 && need2 <= max_tiles2;
  if (!start_in && tid < n_experts) {
    // each chunk's first slot of this expert: its offset plus the counts of the chunks before
    uint32_t at = v[0];
    for (uint32_t b = 0; b < n_chunks; ++b) {
      const uint64_t hi = (uint64_t)b * n_experts + tid;
      const uint32_t cb = hist[hi];
      hist[hi] = at;
      at += cb;
    }
  }
  if (fits && tid < n_experts) {
    if (!start_in) offsets[tid] = v[0];
    uint32_t at1[kNCls], at2[kNCls], base1 = 0, base2 = 0;
#pragma unroll
    for (int k = 0; k < kNCls; ++k) {
      at1[k] = base1 + v[1 + k];
      at2[k] = base2 + v[1 + kNCls + k];
      base1 += tot[1 + k];
      base2 += tot[1 + kNCls + k];
    }
    put_tiles(tiles1, tid, b0, c, tt1, nar1, mid1, at1);
    put_tiles(tiles2, tid, b0, c, tt2, nar2, mid2, at2);
  }
  if (tid == 0) {
    if (!start_in) offsets[n_experts] = tot[0];
    hdr->n_slots = start_in ? n_slots_in : tot[0];
#pragma unroll
    for (int k = 0; k < kNCls; ++k) {
      hdr->n_cls[0][k] = fits ? tot[1 + k] : 0u;
      hdr->n_cls[1][k] = fits ? tot[1 + kNCls + k] : 0u;
    }
    hdr->tx = tx;
    hdr->bad = fits ? 0u : 1u;
  }
}

// The routes form's placement, in two passes over chunks of kPlaceChunk routes (four rounds of
// 256): grouped_hist_kernel counts each expert's routes per chunk, grouped_plan_kernel turns the
// counts into each chunk's first slot per expert, grouped_place_kernel gives every route its slot.
// A route's slot is its expert's offset plus the number of that expert's routes before it, so
// each expert's slots hold its routes in route order, whatever the grid.
constexpr uint32_t kPlaceChunk = 1024;

// Counts of chunk blockIdx.x into hist[chunk][expert]. Also the routes form's ord/run for the
// indices it covers: token t owns entries t k .. t k + k - 1 of ord, in route order (run[t] = t k);
// a route that names no expert of the layer keeps ~0u there (the consumers skip slot numbers past
// the slot count), grouped_place_kernel writes the slot of every other.
__global__ void __launch_bounds__(256) grouped_hist_kernel(const uint32_t* __restrict__ sel, uint32_t n_pairs,
                                                           uint32_t n_tok, uint32_t top_k, uint32_t n_experts,
                                                           uint32_t* __restrict__ hist, uint32_t* __restrict__ run,
                                                           uint32_t* __restrict__ ord) {
  __shared__ uint32_t cnt[AFFX_MAX_EXPERTS];
  const uint32_t b = blockIdx.x, tid = threadIdx.x;
  for (uint32_t e = tid; e < n_experts; e += 256) cnt[e] = 0u;
  __syncthreads();
  uint32_t ev[kPlaceChunk / 256];
#pragma unroll
  for (uint32_t r = 0; r < kPlaceChunk / 256; ++r) {
    const uint32_t i = b * kPlaceChunk + r * 256u + tid;
    ev[r] = i < n_pairs ? sel[i] : ~0u;
  }
#pragma unroll
  for (uint32_t r = 0; r < kPlaceChunk / 256; ++r) {
    const uint32_t i = b * kPlaceChunk + r * 256u + tid;
    if (ev[r] < n_experts)
      atomicAdd(&cnt[ev[r]], 1u);
    else if (i < n_pairs)
      ord[i] = ~0u;
    if (i <= n_tok) run[i] = i * top_k;
  }
  __syncthreads();
  for (uint32_t e = tid; e < n_experts; e += 256) hist[(uint64_t)b * n_experts + e] = cnt[e];
}

// The slots of chunk blockIdx.x. first[chunk][expert] is the chunk's first slot of each expert
// (grouped_plan_kernel). Routes i = chunk start + 256 r + 64 w + lane: within a wave, the lanes of
// the same expert are ranked by one ballot per expert-id bit; the (round, wave) groups are ranked
// by an exclusive scan of their per-expert counts in LDS.
__global__ void __launch_bounds__(256) grouped_place_kernel(const uint32_t* __restrict__ sel,
                                                            const float* __restrict__ w, uint32_t n_pairs,
                                                            uint32_t top_k, uint32_t n_experts,
                                                            const uint32_t* __restrict__ first,
                                                            uint32_t* __restrict__ slot_tok,
                                                            float* __restrict__ slot_w, uint32_t* __restrict__ ord) {
  static_assert(AFFX_MAX_EXPERTS <= 512, "expert ids ranked by 9 ballots");
  constexpr uint32_t NR = kPlaceChunk / 256, NG = NR * 4;  // rounds, (round, wave) groups
  __shared__ uint32_t grp[NG][AFFX_MAX_EXPERTS];
  const uint32_t b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  for (uint32_t q = tid; q < NG * AFFX_MAX_EXPERTS; q += 256) (&grp[0][0])[q] = 0u;
  uint32_t ev[NR], rank[NR];
#pragma unroll
  for (uint32_t r = 0; r < NR; ++r) {
    const uint32_t i = b * kPlaceChunk + r * 256u + tid;
    ev[r] = i < n_pairs ? sel[i] : ~0u;
  }
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (uint32_t r = 0; r < NR; ++r) {
    const bool ok = ev[r] < n_experts;
    const uint64_t m = same_key_lanes<9>(ok ? ev[r] : 0u, ok);
    rank[r] = (uint32_t)__popcll(m & below);
    if (ok && (uint32_t)__builtin_ctzll(m) == lane) grp[r * 4u + wv][ev[r]] = (uint32_t)__popcll(m);
  }
  __syncthreads();
  for (uint32_t e = tid; e < n_experts; e += 256) {
    uint32_t at = 0;
#pragma unroll
    for (uint32_t g = 0; g < NG; ++g) {
      const uint32_t c = grp[g][e];
      grp[g][e] = at;
      at += c;
    }
  }
  __syncthreads();
  const uint32_t* fb = first + (uint64_t)b * n_experts;
#pragma unroll
  for (uint32_t r = 0; r < NR; ++r) {
    if (!(ev[r] < n_experts)) continue;
    const uint32_t i = b * kPlaceChunk + r * 256u + tid;
    const uint32_t pos = fb[ev[r]] + grp[r * 4u + wv][ev[r]] + rank[r];
    slot_tok[pos] = i / top_k;
    slot_w[pos] = w[i];
    ord[i] = pos;
  }
}

// ------------------------------------------------------------------------------------------------
// activation terms: per token an exponent and tx E4M3 terms of every element, in step order
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) grouped_prep_x_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ xlo,
                                                             uint32_t hidden, uint32_t tx,
                                                             const uint32_t* __restrict__ ord,
                                                             const uint32_t* __restrict__ run,
                                                             uint32_t n_slots,
                                                             int32_t* __restrict__ slot_sigma,
                                                             uint8_t* __restrict__ xq,
                                                             uint32_t* __restrict__ zeros,
                                                             uint32_t zero_words) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  if (t == 0)  // the B row of unused columns
    for (uint32_t i = tid; i < zero_words; i += 256) zeros[i] = 0u;
  __shared__ float red[4];
  const int sigma = row_terms<true>(x + (uint64_t)t * hidden, xlo ? xlo + (uint64_t)t * hidden : nullptr, hidden,
                                    tx, xq + (uint64_t)t * tx * hidden, red);
  // the exponent goes to each of the token's slots, for the gate/up epilogue
  const uint32_t r1 = min(run[t + 1], n_slots);
  for (uint32_t i = min(run[t], r1) + tid; i < r1; i += 256) {
    const uint32_t sl = ord[i];
    if (sl < n_slots) slot_sigma[sl] = sigma;
  }
}

// ------------------------------------------------------------------------------------------------
// grouped GEMM: one workgroup = one (expert, token tile) x one row block
// ------------------------------------------------------------------------------------------------
// 8 waves, two per SIMD: on gfx950 one wave's VALU work does not overlap its own MFMAs, but it
// does overlap the other wave's. A wave owns 32 weight rows (two 16-row tiles: gate/up = one gate
// tile and the same rows of up, down = two tiles) against all 192 B columns of the tile (12 MFMA
// column tiles; a token is TX adjacent columns, 16 / TX tokens per column tile). Per MFMA step
// (128 of K):
//   - each wave decodes its own rows' A fragments in registers: one codebook lookup per quad
//     code, reused by 12 MFMAs. The table holds each codebook dword and its half-rotated form
//     (the rotation field of a block selects the table), so a code costs two VALU ops for its
//     address and one for sign and scale. Two interleaved copies (lane parity): on this kernel
//     the VALU, not the LDS bank conflicts, sets the pace, and fewer copies measured as fast as
//     four or eight;
//   - B (192 columns x 128 bytes) sits in LDS, written by direct global->LDS loads two steps at
//     a time, two steps ahead (four buffers, one workgroup barrier per two steps), read by all
//     eight waves; 16-byte chunks are swizzled by column so that
//     the fragment reads of 16 lanes hit 16 distinct bank groups;
//   - the packed weights of the next 1024 columns stream into a register ring, each chunk
//     reloaded as soon as the lookups of the current 1024 columns are past it.
constexpr int kGW = 8;                      // waves per workgroup (two per SIMD)
constexpr int kGRT = 16 / kGW;              // 16-row tiles per wave (a workgroup covers 256 rows)
constexpr int kGT = kGW * 64;
constexpr int kGKC = 2;                     // codebook copies (pre-rotated tables)
constexpr int kGCT = 12;                    // 16-column tiles of B per wave (a wide tile)
constexpr int kGMid = 8;                    // the same for a mid tile
constexpr int kGNarrow = 4;                 // the same for a narrow tile
// A tile of CT column tiles (kGCT, kGMid or kGNarrow): its B columns, the bytes of one B buffer
// (one MFMA step) and the direct-load instructions per wave per step (8 columns each).
template <int CT>
struct GTile {
  static constexpr int kCols = CT * 16;
  static constexpr uint32_t kBuf = kCols * 128;
  static constexpr int kDma = kCols / 8 / kGW;
};

struct GemmArgs {
  const uint8_t* base;
  uint64_t stride;
  uint64_t off[9];
  uint32_t hidden, inter;
  const uint32_t* codebook;
  const GroupedHdr* hdr;
  const Tile* tiles;
  uint32_t max_tiles;       // entries of tiles (allocated; the header says how many are used)
  const uint32_t* slot_tok;
  uint32_t n_sl;              // entries of slot_tok and slot_sigma
  uint32_t n_tok;             // tokens of the batch (a slot's token id is clamped below it)
  const int32_t* slot_sigma;  // activation exponent of the slot's token
  const uint8_t* ws;        // B rows and the zero row, addressed by 32-bit offsets from here
  uint64_t b_off, zero_off;
  uint8_t* aq;              // gate/up output [slot][3][inter], step order
  float* z;                 // down output [slot][hidden]
  float limit;
  int32_t sigma_a;
};


constexpr int kNT = 2;  // cache policy of streamed weights: non-temporal

// One unit in full (fields first, then the code chunks in order): tile t of the code and field
// planes cr, fr.
__device__ __forceinline__ void load_unit_buf(Unit& u, __amdgpu_buffer_rsrc_t cr, __amdgpu_buffer_rsrc_t fr,
                                              uint32_t t, uint32_t lane) {
#pragma unroll
  for (int q = 0; q < 3; ++q)
    u.f[q] = __builtin_amdgcn_raw_buffer_load_b32(fr, lane * 12u, t * kTileFieldBytes + 4u * q, kNT);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(cr, lane * 16u, t * kTileCodeBytes + 1024u * j, kNT);
    u.c[4 * j] = v[0]; u.c[4 * j + 1] = v[1]; u.c[4 * j + 2] = v[2]; u.c[4 * j + 3] = v[3];
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Registers of a unit that the ring reloads at step M (for the next 1024 columns). Step M's
// reloads come before its table reads (those of step M + 1), so a register is reloaded at the
// first step after the last step whose table reads use it: code chunk j = c[4j..4j+3] (chunk 0
// at step 1, 1 at 3, 2 at 4, 3 at 6, 4 at 7) and field dword q (f0 at 2, f1 at 5, f2 at 7). One
// load instruction each: steps 1-6 issue one per unit, step 7 two, step 0 none.
template <int M>
__device__ __forceinline__ void ring_load(Unit& u, __amdgpu_buffer_rsrc_t cr, __amdgpu_buffer_rsrc_t fr, uint32_t t,
                                          uint32_t lane) {
  auto chunk = [&](int j) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(cr, lane * 16u, t * kTileCodeBytes + 1024u * j, kNT);
    u.c[4 * j] = v[0]; u.c[4 * j + 1] = v[1]; u.c[4 * j + 2] = v[2]; u.c[4 * j + 3] = v[3];
  };
  auto field = [&](int q) {
    u.f[q] = __builtin_amdgcn_raw_buffer_load_b32(fr, lane * 12u, t * kTileFieldBytes + 4u * q, kNT);
  };
  if constexpr (M == 1) chunk(0);
  if constexpr (M == 2) field(0);
  if constexpr (M == 3) chunk(1);
  if constexpr (M == 4) chunk(2);
  if constexpr (M == 5) field(1);
  if constexpr (M == 6) chunk(3);
  if constexpr (M == 7) { chunk(4); field(2); }
}

template <int PH, int TX, int CT>
__global__ void __launch_bounds__(kGT, 1) grouped_gemm_kernel(GemmArgs A) {
  constexpr int TPG = 16 / TX;  // tokens per 16-column tile
  constexpr int kHalf = kGRT / 2;  // gate/up: units [0, kHalf) gate, [kHalf, kGRT) the same rows of up
  // Persistent: workgroup b runs the items (row block, token tile) w = b, b + G, b + 2G, ... (G =
  // gridDim.x, a multiple of 8). XCD-aware order: the device hands consecutive workgroups to its
  // 8 XCDs in turn, so workgroup b runs on XCD b % 8 = w % 8 for all of its items. All row blocks
  // of one token tile go to the same XCD (its L2 then holds the tile's activations for all of
  // them), consecutive tiles to different XCDs. Items are in increasing tile order per workgroup,
  // so the first item past the last tile ends the workgroup.
  const uint32_t nrb = PH == 0 ? A.inter / 128u : A.hidden / 256u;  // row blocks
  auto item_of = [&](uint32_t w, uint32_t& rb_, uint32_t& tile_) {
    const uint32_t l = w >> 3;
    rb_ = l % nrb;
    tile_ = (l / nrb) * 8u + (w & 7u);
  };
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t K = PH == 0 ? A.hidden : A.inter;
  const uint32_t nst = K / kTileCols;
  const uint32_t nsteps = nst * 8u;
  // Set-up of the first item in three memory round trips: (1) the codebook, the tile count and
  // the tiles of the first two items (read before it is known to be in use: any index below
  // max_tiles is allocated); (2) the B row of every column, then the first weights; (3) the
  // first two steps of B. Later items find their tile and B rows staged in LDS (see ep_sig), and
  // their first weights and B steps are loaded during the previous item's last 1024 columns (see
  // cont).
  constexpr int kPer = 2048 / kGT;
  uint32_t cbv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) cbv[i] = A.codebook[tid + (uint32_t)kGT * i];
  // this instantiation's tiles: those of its width class, stored after the wider classes' tiles
  constexpr int cls = CT == kGCT ? 0 : CT == kGMid ? 1 : 2;
  const uint32_t* ncls = A.hdr->n_cls[PH];
  const uint32_t n_tiles = ncls[cls];
  const uint32_t first = (cls > 0 ? ncls[0] : 0u) + (cls > 1 ? ncls[1] : 0u);
  // (entries below max_t are allocated: read before it is known whether a tile is in use)
  const uint32_t room = A.max_tiles - min(first, A.max_tiles);
  const Tile* tiles = room ? A.tiles + first : A.tiles;
  const uint32_t max_t = room ? room : 1u;
  uint32_t w = blockIdx.x, rb, tile_id, rbn, tile_n;
  item_of(w, rb, tile_id);
  item_of(w + gridDim.x, rbn, tile_n);
  Tile tl = tiles[tile_id < max_t ? tile_id : 0u];
  Tile tln = tiles[tile_n < max_t ? tile_n : 0u];  // the next item's tile
  if (tile_id >= n_tiles || tl.n == 0) return;  // (a tile in use has n >= 1: the test only makes
                                                // the loads precede the branch, in one round trip)
  bool has_next = tile_n < n_tiles && tln.n != 0;

  __shared__ __align__(16) uint32_t lut_s[Lut<kGKC, true>::kDwords];
  __shared__ __align__(16) uint2 blk_s[16];
  const uint8_t* btbl = reinterpret_cast<const uint8_t*>(blk_s);
  // B of step t in buffer t % 4, written two steps at a time, two steps ahead (four separate
  // arrays: the compiler can then tell the buffers being read from the ones being written)
  __shared__ __align__(16) uint8_t buf0[GTile<CT>::kBuf];
  __shared__ __align__(16) uint8_t buf1[GTile<CT>::kBuf];
  __shared__ __align__(16) uint8_t buf2[GTile<CT>::kBuf];
  __shared__ __align__(16) uint8_t buf3[GTile<CT>::kBuf];
  uint32_t* rowoff = reinterpret_cast<uint32_t*>(buf3);  // set-up only, before buffer 3 is written
  __shared__ __align__(16) uint32_t rowoff_n[GTile<CT>::kCols];  // the next tile's, during the last 1024 columns
  // Staged at the start of each item by direct-to-LDS loads, so that neither the epilogue nor the
  // step to the next item waits for memory: the item's activation exponents (gate/up: one per
  // slot of the tile, 128 entries) and row scales (256 bf16: the 128 gate and 128 up rows, or the
  // 256 down rows), the next item's B rows (gate/up: its slots' tokens) and the tile of the item
  // after it.
  __shared__ __align__(16) uint32_t ep_sig[128];
  __shared__ __align__(16) uint32_t ep_rs[128];
  __shared__ __align__(16) uint32_t ep_tok[128];
  __shared__ __align__(16) uint32_t ep_tile[64];
  const uint8_t* lut = reinterpret_cast<const uint8_t*>(lut_s);
  auto bufsel = [&](int i) -> uint8_t* { return i == 0 ? buf0 : i == 1 ? buf1 : i == 2 ? buf2 : buf3; };

  // ---- per-item state: the expert's planes, this wave's row tiles, the B rows -----------------
  // the wave's 16-row tiles: gate/up = gate tile rt0 (unit 0) and the same rows of up (unit 1);
  // down = two consecutive tiles. Unit r's code/field planes: (c0, f0) for the gate unit or down,
  // (c1, f1) for the up unit.
  const uint64_t cbytes = (uint64_t)(PH == 0 ? A.inter : A.hidden) * code_row_bytes(K);
  const uint64_t fbytes = (uint64_t)(PH == 0 ? A.inter : A.hidden) * field_row_bytes(K);
  const uint8_t* ex;
  __amdgpu_buffer_rsrc_t c0, f0, c1, f1;
  uint32_t rt0;
  auto set_item = [&](const Tile& t, uint32_t rb_) {
    ex = A.base + (uint64_t)t.expert * A.stride;
    c0 = buffer_rsrc(ex + A.off[PH == 0 ? kGateCodes : kDownCodes], (uint32_t)cbytes);
    f0 = buffer_rsrc(ex + A.off[PH == 0 ? kGateFields : kDownFields], (uint32_t)fbytes);
    c1 = buffer_rsrc(ex + A.off[PH == 0 ? kUpCodes : kDownCodes], (uint32_t)cbytes);
    f1 = buffer_rsrc(ex + A.off[PH == 0 ? kUpFields : kDownFields], (uint32_t)fbytes);
    rt0 = PH == 0 ? rb_ * 8u + kHalf * wv : rb_ * 16u + kGRT * wv;
  };
  auto rt_of = [&](int r) -> uint32_t { return PH == 0 ? rt0 + (r % kHalf) : rt0 + r; };
  Unit u[kGRT];
  auto load_units = [&]() {
#pragma unroll
    for (int r = 0; r < kGRT; ++r)
      load_unit_buf(u[r], PH == 0 && r >= kHalf ? c1 : c0, PH == 0 && r >= kHalf ? f1 : f0, rt_of(r) * nst, lane);
  };
  // B row of column tid (threads below GTile<CT>::kCols): a column past the tile's tokens reads the tile's
  // first slot (unconditional load) and gets the zero row
  // (these and the per-item lane values below are derived from an opaque copy of the thread index
  // where they are used: derived once, outside the item loop, they were held across it, spilled,
  // and every reload from scratch memory waited for all the loads in flight)
  auto tid_now = [&]() -> uint32_t {
    uint32_t z = 0u;
    AFFX_PIN(z);  // (the lane count below is made where it is used, from nothing held across)
    return wv * 64u + __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, z));
  };
  const uint32_t bcol_j = (tid >> 4) * TPG + (tid & 15u) / TX;
  auto brow_load = [&](const Tile& t) -> uint32_t {
    const uint32_t bslot = t.slot0 + ((tid < GTile<CT>::kCols && (tid & 15u) < TX * TPG && bcol_j < t.n) ? bcol_j : 0u);
    return PH == 0 ? min(A.slot_tok[bslot], A.n_tok - 1u) : bslot;
  };
  // the same from the tokens staged in ep_tok (slot t.slot0 + j at entry j)
  auto brow_staged = [&](const Tile& t) -> uint32_t {
    const uint32_t tp = tid_now(), bj = (tp >> 4) * TPG + (tp & 15u) / TX;
    const uint32_t j = (tp < GTile<CT>::kCols && (tp & 15u) < TX * TPG && bj < t.n) ? bj : 0u;
    return PH == 0 ? min(ep_tok[j], A.n_tok - 1u) : t.slot0 + j;
  };
  // (B rows are addressed by 32-bit offsets into the workspace, which the host checks fit, so the
  // offsets are computed in 32 bits)
  auto rowoff_store = [&](const Tile& t, uint32_t brow) {
    const uint32_t tp = tid_now(), bj = (tp >> 4) * TPG + (tp & 15u) / TX;
    const bool used = tp < GTile<CT>::kCols && (tp & 15u) < TX * TPG && bj < t.n;
    if (tp < GTile<CT>::kCols)
      rowoff[tp] = used ? (uint32_t)A.b_off + (brow * TX + (tp & 15u) % TX) * K : (uint32_t)A.zero_off;
  };
  auto rowoff_store_next = [&](const Tile& t, uint32_t brow) {
    const uint32_t tp = tid_now(), bj = (tp >> 4) * TPG + (tp & 15u) / TX;
    const bool used = tp < GTile<CT>::kCols && (tp & 15u) < TX * TPG && bj < t.n;
    if (tp < GTile<CT>::kCols)
      rowoff_n[tp] = used ? (uint32_t)A.b_off + (brow * TX + (tp & 15u) % TX) * K : (uint32_t)A.zero_off;
  };
  // DMA lane map: instruction i of wave w writes columns 8b..8b+7 (b = GTile<CT>::kDma w + i), lane l to
  // LDS slot l & 7 of column 8b + (l >> 3); slot p of column col holds global chunk p ^ f(col),
  // f(col) = (c ^ (c >> 3)) & 7 with c = col & 15 (the column within its 16-column tile), that
  // is (col & 7) ^ ((col >> 3) & 1). A fragment read (lane = column c + 16 k-group) then puts lanes
  // 0-7, 8-15 (and so on) on 8 distinct 16-byte bank groups, and lanes 0-15 on 16.
  // (sized for the wide tile, a narrow one uses the first entries: with a size that depends on CT,
  // captured by the lambdas below, ROCm 7.2's hipcc emits no host stub for the kernel)
  uint32_t roff[GTile<kGCT>::kDma];
  auto roff_load = [&]() {
    const uint32_t lp = tid_now() & 63u;
#pragma unroll
    for (int i = 0; i < GTile<CT>::kDma; ++i) {
      const uint32_t col = 8u * (GTile<CT>::kDma * wv + i) + (lp >> 3);
      const uint32_t q = (lp & 7u) ^ ((col & 7u) ^ ((col >> 3) & 1u));
      roff[i] = rowoff[col] + (q << 4);
    }
  };
  auto roff_load_next = [&]() {
    const uint32_t lp = tid_now() & 63u;
#pragma unroll
    for (int i = 0; i < GTile<CT>::kDma; ++i) {
      const uint32_t col = 8u * (GTile<CT>::kDma * wv + i) + (lp >> 3);
      const uint32_t q = (lp & 7u) ^ ((col & 7u) ^ ((col >> 3) & 1u));
      roff[i] = rowoff_n[col] + (q << 4);
    }
  };
  const __amdgpu_buffer_rsrc_t wsr = buffer_rsrc(A.ws, 0xFFFFFFFFu);
  auto dma = [&](uint8_t* buf, uint32_t step) {
#pragma unroll
    for (int i = 0; i < GTile<CT>::kDma; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, AFFX_LDS_PTR(buf + (GTile<CT>::kDma * wv + i) * 1024u), 16, roff[i],
                                               step * 128u, 0, 0);
  };

  // ---- set-up of the first item (B row loads first: the set-up waits for them, and loads
  // complete in issue order; then the weights; the codebook copies while they are in flight) ---
  {
    const uint32_t brow = brow_load(tl);
    __builtin_amdgcn_sched_barrier(0);
    set_item(tl, rb);
    load_units();
    __builtin_amdgcn_sched_barrier(0);
    build_lut<kGKC, kGT, kPer, true>(lut_s, cbv, tid);
    build_blk_tbl(blk_s, tid);
    rowoff_store(tl, brow);
    __syncthreads();
    roff_load();
    dma(buf0, 0);
    dma(buf1, 1);
    __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }

  // epilogue helpers: accumulator lane (c, kg), element v = D[4 kg + v][c]: row 4 kg + v of the
  // row tile, column c. (Every accumulator index is a compile-time constant: a runtime index
  // would put the whole accumulator array in scratch memory.)
  auto terms = [&](float d) -> float {
    const float d1 = row_shl<1>(d);
    if constexpr (TX == 2) {
      return d + d1 * 0.0625f;
    } else {
      const float d2 = row_shl<2>(d);
      return d + d1 * 0.0625f + d2 * 0.00390625f;
    }
  };
  auto bf16x4 = [](uint2 v, float (&o)[4]) {
    o[0] = __uint_as_float(v.x << 16);
    o[1] = __uint_as_float(v.x & 0xFFFF0000u);
    o[2] = __uint_as_float(v.y << 16);
    o[3] = __uint_as_float(v.y & 0xFFFF0000u);
  };
  const float L = A.limit;

  const __amdgpu_buffer_rsrc_t sig_r = buffer_rsrc(A.slot_sigma, 4u * A.n_sl);
  const __amdgpu_buffer_rsrc_t tok_r = buffer_rsrc(A.slot_tok, 4u * A.n_sl);
  const __amdgpu_buffer_rsrc_t tile_r = buffer_rsrc(tiles, (uint32_t)sizeof(Tile) * max_t);
  auto lds4 = [&](__amdgpu_buffer_rsrc_t r, uint32_t* dst, uint32_t byte_off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, AFFX_LDS_PTR(dst), 4, lane * 4u, byte_off, 0, 0);
  };
  for (;;) {
    // ---- staging (one wave each; issued before the steps' loads, so the steps' exact wait
    // counts are unchanged: loads complete in issue order) ----------------------------------------
    {
      uint32_t rb2s, tile2s;
      item_of(w + 2u * gridDim.x, rb2s, tile2s);
      if (wv == 0) {
        if constexpr (PH == 0) {
          lds4(sig_r, ep_sig, 4u * tl.slot0);
          lds4(sig_r, ep_sig + 64, 4u * tl.slot0 + 256u);
        }
      } else if (wv == 1) {
        const __amdgpu_buffer_rsrc_t rs_r =
            buffer_rsrc(ex + A.off[PH == 0 ? kGateRs : kDownRs], 2u * (PH == 0 ? A.inter : A.hidden));
        if constexpr (PH == 0) {
          lds4(rs_r, ep_rs, 256u * rb);
          lds4(buffer_rsrc(ex + A.off[kUpRs], 2u * A.inter), ep_rs + 64, 256u * rb);
        } else {
          lds4(rs_r, ep_rs, 512u * rb);
          lds4(rs_r, ep_rs + 64, 512u * rb + 256u);
        }
      } else if (wv == 2) {
        if constexpr (PH == 0) {
          if (has_next) {
            lds4(tok_r, ep_tok, 4u * tln.slot0);
            lds4(tok_r, ep_tok + 64, 4u * tln.slot0 + 256u);
          }
        }
      } else if (wv == 3) {
        lds4(tile_r, ep_tile, (uint32_t)sizeof(Tile) * (tile2s < max_t ? tile2s : 0u));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // this item's row tiles (set_item moves rt0 to the next item's during the last 1024 columns)
    const uint32_t rt0_cur = rt0;
    auto rt_cur = [&](int r) -> uint32_t { return PH == 0 ? rt0_cur + (r % kHalf) : rt0_cur + r; };
    // The next item's first weights stream into the register ring during this item's last 1024
    // columns, in place of the ring's idle reloads, and its first two steps of B go out at step 6
    // of those columns, so the step to the next item waits for no load (a burst of the next item's
    // loads there or before the epilogue was held by the memory pipeline). Needs the next item's B
    // rows staged (visible after the first barrier, so at least two sets of 1024 columns).
    const bool cont = has_next && nst >= 2u;
    // the lane's table copy, fragment offsets and epilogue position (derived per item: see tid_now)
    const uint32_t lane_p = tid_now() & 63u;
    const uint32_t copy4 = (lane_p & (kGKC - 1)) * 4u;
    const uint32_t c = lane_p & 15, kg = lane_p >> 4;
    const uint32_t bo0 = c * 128u + (((2u * kg) ^ ((c ^ (c >> 3)) & 7u)) << 4);
    const uint32_t bo1 = c * 128u + (((2u * kg + 1u) ^ ((c ^ (c >> 3)) & 7u)) << 4);
    v8i a_cur[kGRT];
#pragma unroll
    for (int r = 0; r < kGRT; ++r) {
      uint32_t raw[8], sx[4];
      lut_lookup_step<kGKC, true>(u[r], lut, btbl, copy4, 0, raw, sx);
      a_cur[r] = lut_finish(raw, sx);
    }
    v4f acc[kGRT][CT];
#pragma unroll
    for (int r = 0; r < kGRT; ++r)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[r][ct] = v4f{0.f, 0.f, 0.f, 0.f};

    // ---- main loop: 1024 columns of K per iteration, eight MFMA steps ---------------------------
    // (each step is instantiated with its index as a constant: the ring loads, the code positions
    // and the wait counts of a step are all fixed at compile time)
    auto step = [&](auto mc, uint32_t s, bool more) {
      constexpr int m = decltype(mc)::value;
      const uint8_t* bcur = bufsel(m & 3);
      // B of steps t + 2 and t + 3, issued at the top of even steps t into the buffers of steps
      // t - 2 and t - 1 (read before the barrier that ended step t - 1): the workgroup then needs
      // one barrier per two steps. Past the last step the loads repeat the last step's B into
      // buffers nobody reads again, so the count of loads in flight is the same on every path.
      if constexpr ((m & 1) == 0) {
        const uint32_t t2 = s * 8u + m + 2u, t3 = t2 + 1u;
        // (at step 6 of the last 1024 columns: the next item's steps 0 and 1, which go to buffers
        // 0 and 1 as those of steps t + 2 and t + 3 would)
        const bool nx = m == 6 && !more && cont;
        if constexpr (m == 6) {
          if (nx) roff_load_next();
        }
        dma(bufsel((m + 2) & 3), nx ? 0u : t2 < nsteps ? t2 : nsteps - 1u);
        dma(bufsel((m + 3) & 3), nx ? 1u : t3 < nsteps ? t3 : nsteps - 1u);
      }
      __builtin_amdgcn_sched_barrier(0);
      // ring loads for the next 1024 columns; after the last ones, the same loads of tile 0 (hot
      // in the cache, read by every workgroup): their registers are not read again, and issuing
      // them keeps the count of loads in flight the same on every path
      if constexpr (m != 0) {
#pragma unroll
        for (int r = 0; r < kGRT; ++r)
          ring_load<m>(u[r], PH == 0 && r >= kHalf ? c1 : c0, PH == 0 && r >= kHalf ? f1 : f0,
                       more ? rt_of(r) * nst + s + 1 : cont ? rt_of(r) * nst : 0u, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
      // The step is 12 groups, one per B column tile: the tile's two fragment reads go out two
      // groups ahead, its MFMAs (one per row tile) are each followed by a share of the VALU work of
      // the next step (groups 4-5: code addresses and table reads of unit g - 4; groups 8-9: the
      // sign/scale finish of unit g - 8, whose reads were issued four groups earlier). The VALU of
      // one wave runs while the matrix core works through the other wave's MFMAs. The groups are
      // placed so that the table reads and the next A fragments are live for a third of the step
      // only: with two waves per SIMD a wave has 256 registers, accumulators included. (Step 0 of
      // the next 1024 columns after step 7: the ring has reloaded every register those reads use.)
      constexpr int mn = (m + 1) & 7;
      constexpr int kLook = CT >= 12 ? 4 : CT >= 8 ? 2 : 0, kFin = CT >= 12 ? 8 : CT >= 8 ? 5 : 2;
      uint32_t rawn[kGRT][8], sxn[kGRT][4];
      v8i a_next[kGRT];
      auto bread = [&](int ct) -> v8i {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(bcur + ct * 2048 + bo0);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(bcur + ct * 2048 + bo1);
        v8i b;
        b[0] = (int)lo[0]; b[1] = (int)lo[1]; b[2] = (int)lo[2]; b[3] = (int)lo[3];
        b[4] = (int)hi[0]; b[5] = (int)hi[1]; b[6] = (int)hi[2]; b[7] = (int)hi[3];
        return b;
      };
      v8i bq0 = bread(0), bq1 = bread(1);
      static_for<0, CT>([&](auto cc) {
        constexpr int ct = decltype(cc)::value;
        v8i bq2;
        if constexpr (ct + 2 < CT) bq2 = bread(ct + 2);
#pragma unroll
        for (int r = 0; r < kGRT; ++r) acc[r][ct] = mfma(a_cur[r], bq0, acc[r][ct]);
        if constexpr (ct >= kLook && ct < kLook + kGRT) {
          pin_step<mn>(u[ct - kLook]);
          lut_lookup<kGKC, mn, true>(u[ct - kLook], lut, btbl, copy4, rawn[ct - kLook], sxn[ct - kLook]);
        } else if constexpr (ct >= kFin && ct < kFin + kGRT) {
          a_next[ct - kFin] = lut_finish(rawn[ct - kFin], sxn[ct - kFin]);
          AFFX_PIN(a_next[ct - kFin]);  // computed here, not sunk into the next step
        }
        // {one MFMA, then up to 12 VALU} per row tile, then the LDS reads (8, 12, 16, 24 and no
        // pattern measured within about 1 % of each other)
#pragma unroll
        for (int i = 0; i < kGRT; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 10, 0);
        __builtin_amdgcn_sched_barrier(0);
        bq0 = bq1;
        if constexpr (ct + 2 < CT) bq1 = bq2;
      });
      // the accumulators are materialised here (else the compiler sinks every MFMA below all
      // eight steps' table reads and holds those in registers). They stay in VGPRs: a kernel that
      // names no AGPR gets its whole register budget as VGPRs, where one that does is split half
      // and half, and the other half is then too small for the rest of the step.
#pragma unroll
      for (int r = 0; r < kGRT; ++r)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) AFFX_PIN(acc[r][ct]);
#pragma unroll
      for (int r = 0; r < kGRT; ++r) a_cur[r] = a_next[r];
      // After an odd step t: the B of steps t + 1 and t + 2 (issued at the top of step t - 1) is in
      // LDS once every wave's loads up to them have landed. Loads complete in issue order, so at
      // most the loads issued after them may still be outstanding: the ring loads of steps t - 1
      // and t (2 units x {0,1,1,1,1,1,1,2} by step).
      if constexpr ((m & 1) == 1) {
        constexpr int c[8] = {0, 1, 1, 1, 1, 1, 1, 2};
        constexpr int k = kGRT * (c[m - 1] + c[m]);
        __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(k));
        __builtin_amdgcn_s_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    for (uint32_t s = 0; s < nst; ++s) {
      const bool more = s + 1 < nst;
      if (!more && cont) {
        // the next item's planes and B-row offsets (published by the barrier of step 1)
        rowoff_store_next(tln, brow_staged(tln));
        set_item(tln, rbn);
      }
      step(IConst<0>{}, s, more);
      step(IConst<1>{}, s, more);
      step(IConst<2>{}, s, more);
      step(IConst<3>{}, s, more);
      step(IConst<4>{}, s, more);
      step(IConst<5>{}, s, more);
      step(IConst<6>{}, s, more);
      step(IConst<7>{}, s, more);
    }
    // every wave is past its last B read; step 7 waited for every direct-to-LDS load (the next
    // item's first B steps included), and the ring's last loads may stay in flight
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- epilogue inputs, from the staging in LDS -------------------------------------------
    // (gate/up: the activation exponent of the lane's token in each column tile, columns past the
    // tile's tokens read its last token and store nothing; the row scales. Down: row scales.)
    const bool next = has_next;
    int sig[PH == 0 ? CT : 1];
    uint2 rgw[kHalf], ruw[kHalf], rdw[kGRT];
    if constexpr (PH == 0) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const uint32_t j = ct * TPG + c / TX;
        sig[ct] = (int)ep_sig[j < tl.n ? j : tl.n - 1u];
      }
#pragma unroll
      for (int p = 0; p < kHalf; ++p) {
        const uint32_t loc = (rt_cur(p) - rb * 8u) * 16u + 4u * kg;  // row within the gate/up row block
        rgw[p] = *reinterpret_cast<const uint2*>(ep_rs + loc / 2);
        ruw[p] = *reinterpret_cast<const uint2*>(ep_rs + 64 + loc / 2);
      }
    } else {
#pragma unroll
      for (int r = 0; r < kGRT; ++r)
        rdw[r] = *reinterpret_cast<const uint2*>(ep_rs + ((rt_cur(r) - rb * 16u) * 16u + 4u * kg) / 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    // this item's tile, kept for its epilogue
    const Tile tl_cur = tl;
    uint32_t brow2 = 0;
    if (next && !cont) brow2 = brow_staged(tln);
    __builtin_amdgcn_sched_barrier(0);

    // ---- epilogue arithmetic and stores ------------------------------------------------------
    // Gate/up: the SwiGLU terms go to LDS first, term t of the tile's token j at row x of the row
    // block (x < 128) at stg(t) + j * 128 + x (terms 0-1 in buffer 2, term 2 in buffer 3 past the
    // B-row offsets the next item writes there; both buffers are free once the steps are done),
    // and then out in 16-byte pieces: each (token, term) is 128 bytes of the output row, four runs
    // of 32 at a 128-byte stride in the down GEMM's step order. (Written from the accumulator
    // lanes, two or four bytes per lane and term: 36 narrow stores per wave, whose
    // acknowledgements the next item then waited for.)
    constexpr uint32_t kTT = CT * TPG;  // tokens of a tile of this class
    auto stg = [&](uint32_t t) -> uint8_t* { return t < 2 ? buf2 + t * kTT * 128u : buf3 + 1024u; };
    if constexpr (PH == 0) {
      static_for<0, kHalf>([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        const uint32_t row0 = rt_cur(p) * 16u + 4u * kg;
        float rg[4], ru[4];
        bf16x4(rgw[p], rg);
        bf16x4(ruw[p], ru);
        const uint32_t xloc = row0 - rb * 128u;  // the row within the row block
        static_for<0, CT>([&](auto cc) {
          constexpr int ct = decltype(cc)::value;
          if (ct * TPG >= tl_cur.n) return;  // no token in this column tile (the same for the whole wave)
          float sg[4], su[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            sg[v] = terms(acc[p][ct][v]);
            su[v] = terms(acc[p + kHalf][ct][v]);
          }
          const uint32_t j = ct * TPG + c / TX;
          if constexpr (TX == 2) {
            // the lane pair (2i, 2i + 1) shares token i's four rows: the even lane (whose
            // combined terms these are) keeps rows 0-1 and hands rows 2-3 to the odd lane, so
            // every lane runs the SwiGLU and the term split on two values
            const bool odd = (c & 1u) != 0;
            float g2[2], u2[2];
#pragma unroll
            for (int v = 0; v < 2; ++v) {
              const float gu = row_shr<1>(sg[v + 2]), uu = row_shr<1>(su[v + 2]);
              g2[v] = odd ? gu : sg[v];
              u2[v] = odd ? uu : su[v];
            }
            if (j < tl_cur.n) {
              float a2[2];
#pragma unroll
              for (int v = 0; v < 2; ++v) {
                float gv = ldexpf(g2[v], -sig[ct]) * (odd ? rg[v + 2] : rg[v]);
                float uv = ldexpf(u2[v], -sig[ct]) * (odd ? ru[v + 2] : ru[v]);
                gv = (L < gv) ? L : gv;  // SwiGLU with the asymmetric clamp: src/engine/ops.cpp:47-60
                const float lo = (-L < uv) ? uv : -L;
                uv = (lo < L) ? lo : L;
                const float e = __builtin_amdgcn_exp2f(-gv * 1.44269504f);
                a2[v] = ldexpf(gv * __builtin_amdgcn_rcpf(1.0f + e) * uv, A.sigma_a);
              }
              uint32_t o0, o1, o2;
              split3x2(a2[0], a2[1], o0, o1, o2);
              const uint32_t at = j * 128u + xloc + (odd ? 2u : 0u);
              *reinterpret_cast<uint16_t*>(stg(0) + at) = (uint16_t)o0;
              *reinterpret_cast<uint16_t*>(stg(1) + at) = (uint16_t)o1;
              *reinterpret_cast<uint16_t*>(stg(2) + at) = (uint16_t)o2;
            }
          } else if (c % TX == 0 && c < TX * TPG && j < tl_cur.n) {
            float a[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              float gv = ldexpf(sg[v], -sig[ct]) * rg[v];
              float uv = ldexpf(su[v], -sig[ct]) * ru[v];
              gv = (L < gv) ? L : gv;  // SwiGLU with the asymmetric clamp: src/engine/ops.cpp:47-60
              const float lo = (-L < uv) ? uv : -L;
              uv = (lo < L) ? lo : L;
              // (hardware exp2 and reciprocal: a few ulp, far inside the path's tolerance, against
              // some thirty VALU ops per element for expf and an IEEE division; gv -> -inf gives
              // exp -> inf, reciprocal 0, a signed zero)
              const float e = __builtin_amdgcn_exp2f(-gv * 1.44269504f);
              a[v] = ldexpf(gv * __builtin_amdgcn_rcpf(1.0f + e) * uv, A.sigma_a);
            }
            uint32_t o0, o1, o2;
            split3x4(a[0], a[1], a[2], a[3], o0, o1, o2);
            const uint32_t at = j * 128u + xloc;
            *reinterpret_cast<uint32_t*>(stg(0) + at) = o0;
            *reinterpret_cast<uint32_t*>(stg(1) + at) = o1;
            *reinterpret_cast<uint32_t*>(stg(2) + at) = o2;
          }
        });
      });
      __syncthreads();
      // out: piece q (16 bytes) of (token j, term t), k = (t n + j) 8 + q
      const uint32_t n = tl_cur.n, d0 = kperm(rb * 128u);
      const uint32_t tp = tid_now();
      for (uint32_t k = tp; k < n * 24u; k += kGT) {
        const uint32_t q = k & 7u, jt = k >> 3, t = jt / n, j = jt - t * n;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg(t) + j * 128u + q * 16u);
        *reinterpret_cast<u32x4*>(A.aq + ((uint64_t)(tl_cur.slot0 + j) * 3 + t) * A.inter + d0 + (q >> 1) * 128u +
                                  (q & 1u) * 16u) = v;
      }
    } else {
      static_for<0, kGRT>([&](auto rc) {
        constexpr int r = decltype(rc)::value;
        const uint32_t row0 = rt_cur(r) * 16u + 4u * kg;
        float rd[4];
        bf16x4(rdw[r], rd);
        static_for<0, CT>([&](auto cc) {
          constexpr int ct = decltype(cc)::value;
          if (ct * TPG >= tl_cur.n) return;  // no token in this column tile (the same for the whole wave)
          float sd[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) sd[v] = terms(acc[r][ct][v]);
          const uint32_t j = ct * TPG + c / TX;
          if (c % TX == 0 && c < TX * TPG && j < tl_cur.n) {
            float4 o;
            o.x = ldexpf(sd[0], -A.sigma_a) * rd[0];
            o.y = ldexpf(sd[1], -A.sigma_a) * rd[1];
            o.z = ldexpf(sd[2], -A.sigma_a) * rd[2];
            o.w = ldexpf(sd[3], -A.sigma_a) * rd[3];
            *reinterpret_cast<float4*>(A.z + (uint64_t)(tl_cur.slot0 + j) * A.hidden + row0) = o;
          }
        });
      });
    }
    if (!next) break;

    // ---- next item's weights and first two steps of B; the tile of the item after it (staged,
    // read before the next item's staging overwrites it) -----------------------------------------
    Tile tl3;
    tl3.expert = __builtin_amdgcn_readfirstlane(ep_tile[0]);
    tl3.slot0 = __builtin_amdgcn_readfirstlane(ep_tile[1]);
    tl3.n = __builtin_amdgcn_readfirstlane(ep_tile[2]);
    if (!cont) {
      set_item(tln, rbn);
      load_units();
      rowoff_store(tln, brow2);
      __syncthreads();
      roff_load();
      dma(buf0, 0);
      dma(buf1, 1);
    }
    w += gridDim.x;
    rb = rbn;
    tl = tln;
    item_of(w + gridDim.x, rbn, tile_n);
    tln = tl3;
    has_next = tile_n < n_tiles && tln.n != 0;
    __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }
}

// y[t][h] (+)= sum_i wt[ord[i]] * z[ord[i]][h] over token t's slots i = run[t] .. run[t+1]-1, in
// that order (the routes-in entry lists a token's slots in route order).
__global__ void __launch_bounds__(256) grouped_combine_kernel(const float* __restrict__ z,
                                                              const uint32_t* __restrict__ ord,
                                                              const uint32_t* __restrict__ run,
                                                              const float* __restrict__ slot_w,
                                                              uint32_t n_slots, uint32_t hidden,
                                                              float* __restrict__ y, int accumulate) {
  const uint32_t t = blockIdx.y;
  const uint32_t h = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= hidden) return;
  float4 acc = accumulate ? *reinterpret_cast<const float4*>(y + (uint64_t)t * hidden + h)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
  const uint32_t r1 = min(run[t + 1], n_slots);
  for (uint32_t i = min(run[t], r1); i < r1; ++i) {
    const uint32_t s = ord[i];
    if (s >= n_slots) continue;
    const float wt = slot_w[s];
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


struct GroupedWs {
  uint64_t hdr, offsets, run, slot_tok, slot_w, ord, hist, tiles1, tiles2, sigma, zeros, xq, aq, z, total;
  uint32_t max_tiles1, max_tiles2;
};

// tokens per workgroup tile: kGCT column tiles of 16 / terms tokens each
uint32_t tile_tokens(uint32_t terms) { return kGCT * (16 / terms); }

// chunks of the routes form's placement: they cover the routes and the run entries 0 .. T
uint64_t place_chunks(uint32_t T, uint64_t P) {
  const uint64_t n = P > T ? P : (uint64_t)T + 1;
  return (n + kPlaceChunk - 1) / kPlaceChunk;
}

// T tokens, room for P slots (the routes form: T * top_k)
GroupedWs grouped_ws(uint32_t T, uint64_t P, uint32_t E, uint32_t hidden, uint32_t inter, uint32_t tx) {
  GroupedWs w;
  const uint32_t tt1 = tile_tokens(tx), tt2 = tile_tokens(3);
  w.max_tiles1 = (uint32_t)(P / tt1 + E + 1);
  w.max_tiles2 = (uint32_t)(P / tt2 + E + 1);
  uint64_t o = 0;
  w.hdr = o; o += a256(sizeof(GroupedHdr));
  w.offsets = o; o += a256(4ull * (AFFX_MAX_EXPERTS + 1));
  w.run = o; o += a256(4ull * ((uint64_t)T + 1));
  w.slot_tok = o; o += a256(4 * P);
  w.slot_w = o; o += a256(4 * P);
  w.ord = o; o += a256(4 * P);
  w.hist = o; o += a256(4ull * place_chunks(T, P) * E);
  w.tiles1 = o; o += a256(sizeof(Tile) * w.max_tiles1);
  w.tiles2 = o; o += a256(sizeof(Tile) * w.max_tiles2);
  w.sigma = o; o += a256(4 * P);  // per slot
  w.zeros = o; o += a256(hidden > inter ? hidden : inter);
  w.xq = o; o += a256((uint64_t)T * tx * hidden);
  w.aq = o; o += a256(P * 3 * inter);
  w.z = o; o += a256(P * 4 * hidden);
  w.total = o;
  return w;
}

// The two entries' shared body. Routes form (sel != null): plan, run and place build the slot list
// on the device from the routes. Slot-list form: the caller's expert ranges (start), tok, wt, ord
// and run; only the tiles are built here.
int grouped_body(const affx_layer* L, const void* x, const void* x_lo, uint32_t T, const uint32_t* sel,
                 const float* w, uint32_t K, const uint32_t* start, const uint32_t* tok, const float* wt,
                 const uint32_t* ord, const uint32_t* run, uint32_t n_slots, float* y, int accumulate,
                 void* ws, size_t ws_bytes, void* stream, const char* what) {
  if (!L || !x || !y || !ws || !L->base || !L->codebook) return set_error(AFFX_ERR_ARG, "%s: null pointer", what);
  if (L->n_experts == 0 || L->n_experts > AFFX_MAX_EXPERTS)
    return set_error(AFFX_DECLINED, "%s: n_experts must be 1..%d", what, AFFX_MAX_EXPERTS);
  if (L->hidden % kTileCols || L->inter % kTileCols || L->hidden == 0 || L->inter == 0 ||
      L->hidden > 8192 || L->inter > 8192)
    return set_error(AFFX_DECLINED, "%s: hidden and inter must be multiples of 1024, at most 8192", what);
  if (!(L->swiglu_limit > 0.f) || L->swiglu_limit > 1e6f)
    return set_error(AFFX_DECLINED, "%s: needs a SwiGLU clamp limit in (0, 1e6]", what);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(x_lo)) & 15u)
    return set_error(AFFX_ERR_ARG, "%s: x and x_lo must be 16-byte aligned", what);
  const uint32_t tx = x_lo ? 3 : 2;
  const uint64_t P = sel ? (uint64_t)T * K : n_slots;
  const GroupedWs lay = grouped_ws(T, P, L->n_experts, L->hidden, L->inter, tx);
  // the GEMM addresses its B rows with 32-bit offsets into the workspace
  if (P > (1ull << 31) || lay.aq + P * 3 * L->inter > (1ull << 32))
    return set_error(AFFX_DECLINED, "%s: batch too large (split it)", what);
  if (ws_bytes < lay.total)
    return set_error(AFFX_ERR_ARG, "%s: workspace %zu < %llu bytes", what, ws_bytes, (unsigned long long)lay.total);
  uint64_t off9[9];
  const uint64_t stride = affx_expert_layout(L->hidden, L->inter, off9, nullptr);
  if (L->stride < stride) return set_error(AFFX_ERR_ARG, "%s: layer stride below expert size", what);

  uint8_t* b = (uint8_t*)ws;
  hipStream_t s = (hipStream_t)stream;
  const uint32_t* slot_tok = sel ? (const uint32_t*)(b + lay.slot_tok) : tok;
  const float* slot_w = sel ? (const float*)(b + lay.slot_w) : wt;
  const uint32_t* ord_d = sel ? (const uint32_t*)(b + lay.ord) : ord;
  const uint32_t* run_d = sel ? (const uint32_t*)(b + lay.run) : run;
  GemmArgs A;
  A.base = (const uint8_t*)L->base;
  A.stride = L->stride;
  for (int i = 0; i < 9; ++i) A.off[i] = off9[i];
  A.hidden = L->hidden;
  A.inter = L->inter;
  A.codebook = (const uint32_t*)L->codebook;
  A.hdr = (const GroupedHdr*)(b + lay.hdr);
  A.slot_tok = slot_tok;
  A.n_sl = (uint32_t)P;
  A.n_tok = T;
  A.slot_sigma = (const int32_t*)(b + lay.sigma);
  A.ws = b;
  A.zero_off = lay.zeros;
  A.aq = b + lay.aq;
  A.z = (float*)(b + lay.z);
  A.limit = L->swiglu_limit;
  A.sigma_a = 7 - ilogbf(L->swiglu_limit * L->swiglu_limit);

  const uint32_t tt1 = tile_tokens(tx), tt2 = tile_tokens(3);
  const uint32_t Pp = sel ? T * K : 0u;
  // an expert's partial last tile is narrow (mid) when its tokens fill at most kGNarrow (kGMid)
  // column tiles
  const uint32_t nar1 = kGNarrow * (16 / tx), nar2 = kGNarrow * (16 / 3);
  const uint32_t mid1 = kGMid * (16 / tx), mid2 = kGMid * (16 / 3);
  const uint32_t nch = sel ? (uint32_t)place_chunks(T, Pp) : 0u;
  if (sel) {
    hipLaunchKernelGGL(grouped_hist_kernel, dim3(nch), dim3(256), 0, s, sel, Pp, T, K, L->n_experts,
                       (uint32_t*)(b + lay.hist), (uint32_t*)(b + lay.run), (uint32_t*)(b + lay.ord));
    if (int rc0 = check_launch("grouped_hist_kernel")) return rc0;
  }
  hipLaunchKernelGGL(grouped_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, (uint32_t*)(b + lay.hist), nch,
                     L->n_experts, tt1, tt2, nar1,
                     nar2, mid1, mid2, tx, sel ? nullptr : start, sel ? 0u : n_slots, lay.max_tiles1, lay.max_tiles2,
                     (GroupedHdr*)(b + lay.hdr), (uint32_t*)(b + lay.offsets), (Tile*)(b + lay.tiles1),
                     (Tile*)(b + lay.tiles2));
  int rc = check_launch("grouped_plan_kernel");
  if (rc) return rc;
  if (sel) {
    hipLaunchKernelGGL(grouped_place_kernel, dim3(nch), dim3(256), 0, s, sel, w, Pp, K, L->n_experts,
                       (const uint32_t*)(b + lay.hist), (uint32_t*)(b + lay.slot_tok), (float*)(b + lay.slot_w),
                       (uint32_t*)(b + lay.ord));
    if ((rc = check_launch("grouped_place_kernel"))) return rc;
  }
  const uint32_t n_sl = (uint32_t)P;  // slot indices are below this (the routes form's taken slots too)
  const uint32_t zmax = L->hidden > L->inter ? L->hidden : L->inter;
  hipLaunchKernelGGL(grouped_prep_x_kernel, dim3(T), dim3(256), 0, s, (const uint16_t*)x, (const uint16_t*)x_lo,
                     L->hidden, tx, ord_d, run_d, n_sl, (int32_t*)(b + lay.sigma), b + lay.xq,
                     (uint32_t*)(b + lay.zeros), zmax / 4);
  if ((rc = check_launch("grouped_prep_x_kernel"))) return rc;
  // gate/up: 128 gate + 128 up rows per item; down: 256 rows. Items (row block, tile), the tile
  // count rounded up to a multiple of the 8 XCDs (see the kernel's order), run by a persistent
  // grid of one workgroup per CU (a multiple of 8), or fewer when there are fewer items
  int dev = 0, cus = 0;
  if ((rc = check_hip(hipGetDevice(&dev), "hipGetDevice"))) return rc;
  if ((rc = check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute")))
    return rc;
  const uint32_t gmax = cus >= 8 ? (uint32_t)cus / 8u * 8u : 8u;
  // (the mid and narrow tiles: at most one per expert)
  auto grid = [&](uint32_t row_blocks, uint32_t tiles) {
    const uint32_t items = row_blocks * ((tiles + 7) / 8 * 8);
    return items < gmax ? items : gmax;
  };
  const uint32_t E8 = L->n_experts < lay.max_tiles1 ? L->n_experts : lay.max_tiles1;
  A.tiles = (const Tile*)(b + lay.tiles1);
  A.max_tiles = lay.max_tiles1;
  A.b_off = lay.xq;
  const uint32_t g1 = grid(L->inter / 128, lay.max_tiles1), gn1 = grid(L->inter / 128, E8);
  if (tx == 2) {
    hipLaunchKernelGGL((grouped_gemm_kernel<0, 2, kGCT>), dim3(g1), dim3(kGT), 0, s, A);
    hipLaunchKernelGGL((grouped_gemm_kernel<0, 2, kGMid>), dim3(gn1), dim3(kGT), 0, s, A);
    hipLaunchKernelGGL((grouped_gemm_kernel<0, 2, kGNarrow>), dim3(gn1), dim3(kGT), 0, s, A);
  } else {
    hipLaunchKernelGGL((grouped_gemm_kernel<0, 3, kGCT>), dim3(g1), dim3(kGT), 0, s, A);
    hipLaunchKernelGGL((grouped_gemm_kernel<0, 3, kGMid>), dim3(gn1), dim3(kGT), 0, s, A);
    hipLaunchKernelGGL((grouped_gemm_kernel<0, 3, kGNarrow>), dim3(gn1), dim3(kGT), 0, s, A);
  }
  if ((rc = check_launch("grouped_gemm_kernel (gate/up)"))) return rc;
  A.tiles = (const Tile*)(b + lay.tiles2);
  A.max_tiles = lay.max_tiles2;
  A.b_off = lay.aq;
  const uint32_t g2 = grid(L->hidden / 256, lay.max_tiles2), gn2 = grid(L->hidden / 256, E8);
  hipLaunchKernelGGL((grouped_gemm_kernel<1, 3, kGCT>), dim3(g2), dim3(kGT), 0, s, A);
  hipLaunchKernelGGL((grouped_gemm_kernel<1, 3, kGMid>), dim3(gn2), dim3(kGT), 0, s, A);
  hipLaunchKernelGGL((grouped_gemm_kernel<1, 3, kGNarrow>), dim3(gn2), dim3(kGT), 0, s, A);
  if ((rc = check_launch("grouped_gemm_kernel (down)"))) return rc;
  hipLaunchKernelGGL(grouped_combine_kernel, dim3((L->hidden / 4 + 255) / 256, T), dim3(256), 0, s,
                     (const float*)(b + lay.z), ord_d, run_d, slot_w, n_sl, L->hidden, y, accumulate);
  return check_launch("grouped_combine_kernel");
}

}  // namespace

extern "C" {

size_t affx_grouped_workspace_size(uint32_t n_tok, uint32_t top_k, uint32_t n_experts,
                                   uint32_t hidden, uint32_t inter) {
  // sized for the 3-term gate/up input (x with a low part), the larger layout
  return (size_t)grouped_ws(n_tok, (uint64_t)n_tok * top_k, n_experts, hidden, inter, 3).total;
}

int affx_expert_ffn_grouped(const affx_layer* L, const void* x, const void* x_lo, uint32_t T,
                            const uint32_t* sel, const float* w, uint32_t K, float* y,
                            int accumulate, void* ws, size_t ws_bytes, void* stream) {
  if (!sel || !w) return set_error(AFFX_ERR_ARG, "ffn_grouped: null pointer");
  if (T == 0) return AFFX_OK;
  if (K == 0 || K > AFFX_MAX_TOPK)
    return set_error(AFFX_DECLINED, "ffn_grouped: top_k must be 1..%d", AFFX_MAX_TOPK);
  return grouped_body(L, x, x_lo, T, sel, w, K, nullptr, nullptr, nullptr, nullptr, nullptr, 0, y, accumulate, ws,
                      ws_bytes, stream, "ffn_grouped");
}

int affx_expert_ffn_grouped_slots(const affx_layer* L, const void* x, const void* x_lo, uint32_t T,
                                  const uint32_t* expert_start, const uint32_t* tok, const float* wt,
                                  const uint32_t* ord, const uint32_t* run, uint32_t n_slots, float* y,
                                  int accumulate, void* ws, size_t ws_bytes, void* stream) {
  if (!expert_start || !tok || !wt || !ord || !run) return set_error(AFFX_ERR_ARG, "ffn_grouped_slots: null pointer");
  if (T == 0) return AFFX_OK;
  return grouped_body(L, x, x_lo, T, nullptr, nullptr, 0, expert_start, tok, wt, ord, run, n_slots, y, accumulate,
                      ws, ws_bytes, stream, "ffn_grouped_slots");
}

}  // extern "C"
