// The reference's single-matrix W8A8 GEMM over tiles of routed tokens, for a caller that drives
// its batch pipeline step by step (expert_gemm_wmma_hip, src/gpu/expert_kernel_hip.h:217-228;
// kernel src/gpu/expert_kernel.hip:364-825, host 3018-3062). For every tile (one expert matrix,
// nt <= 64 tokens of the chunk) and every row r:
//   y[r][j] = bf16(rs[r]) * wscale * out,  out = fma-fold over the 128-column blocks kb, in order,
//             of raw_kb * xs[t][kb],  raw_kb = sum over the block of W8[r][k] * x8[t][k]
// (expert_kernel.hip:808-818 for the fold, 820-837 for the row scale), t = tok ? tok[j] : j. W8 is
// the weight's E4M3 value without its row scale, x8 the E4M3 activation, xs its f32 scale per
// (token, 128-column block).
//
// Here a workgroup is four waves, 64 rows of one tile; a wave walks the column tiles of its 16-row
// wave tile and decodes each into eight MFMA A fragments (the decode's LDS codebook and step
// order). One MFMA step's 128 K values span four 128-column blocks (lane group g holds 32 columns
// of the tile's segment g), so to keep the blocks' sums apart the B operand places the columns of
// group g of a token in B column 4 (token of the quad) + g and zeros elsewhere: one MFMA gives,
// for four tokens, each group's partial, steps 0-3 completing block 2g of the tile and steps 4-7
// block 2g + 1. A (row, token)'s eight partials then sit in one lane quad, and every lane of the
// quad folds them in block order (DPP quad broadcasts). The tile's activation rows (1024 bytes a
// token) and their block scales are loaded straight into LDS per column tile, up to 32 tokens a
// pass, while the wave decodes its A fragments.
#include "affx_lut.h"

namespace affx {

constexpr int kW8Waves = 4;
constexpr int kW8T = kW8Waves * 64;
constexpr int kW8KC = 2;              // codebook copies
constexpr uint32_t kW8MaxTok = 64;    // the reference's kExpertWmmaTok (expert_kernel_hip.h:195)
constexpr uint32_t kW8Row = kTileCols + 16u;  // LDS bytes of one staged token row (padded)

struct W8a8Args {
  const affx_expert_tile* tiles;
  const uint8_t* x8;
  const float* xs;
  const uint32_t* codebook;
  uint32_t rows, cols;
  float wscale;
  int y_bf16;
};

__device__ __forceinline__ uint16_t w8_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// value of lane G of this lane's quad (DPP quad_perm [G, G, G, G])
template <int G>
__device__ __forceinline__ float quad_lane(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), G * 0x55, 0xF, 0xF, false));
}

// NQ: token quads of the launch (4 NQ tokens, the launch's max_nt rounded up); the tokens are
// staged in passes of at most kW8Pass
constexpr uint32_t kW8Pass = 32;

template <int NQ>
__global__ void __launch_bounds__(kW8T) w8a8_gemm_kernel(W8a8Args A) {
  constexpr int NP = (4 * NQ + (int)kW8Pass - 1) / (int)kW8Pass;  // passes
  constexpr int QP = NQ / NP;                                        // quads a pass
  AFFX_DYN_LDS(lds);  // xb [4 QP][kW8Row] activation rows of the pass, then xsl [4 x 64] f32 scales
  uint8_t* xb = lds;
  float* xsl = reinterpret_cast<float*>(lds + 4u * QP * kW8Row);
  __shared__ __align__(16) uint32_t lut_s[Lut<kW8KC, true>::kDwords];
  const uint8_t* lut = reinterpret_cast<const uint8_t*>(lut_s);
  // one-dimensional grid: tile-major, then 64-row blocks
  const uint32_t nrb = (A.rows / kTileRows + kW8Waves - 1) / kW8Waves;
  const uint32_t tile = blockIdx.x / nrb, rb = blockIdx.x - tile * nrb;
  const affx_expert_tile T = A.tiles[tile];
  const uint32_t ntok = T.nt < 4u * NQ ? T.nt : 4u * NQ;
  if (ntok == 0) return;  // a pad (the whole workgroup returns)
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t c = lane & 15, kg = lane >> 4, copy4 = ((lane >> 1) & (kW8KC - 1)) * 4u;
  const uint32_t nct = A.cols / kTileCols, nkb = A.cols / 128u;
  const uint32_t rt = rb * kW8Waves + wv;
  const bool rows_ok = rt * kTileRows < A.rows;
  const uint32_t* tok = T.tok;
  const uint8_t* codes = reinterpret_cast<const uint8_t*>(T.codes);
  const uint8_t* fields = reinterpret_cast<const uint8_t*>(T.fields);

  uint32_t cbv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cbv[i] = A.codebook[tid + (uint32_t)i * kW8T];
  // the lane's four accumulator rows' scales, times wscale (the reference's order)
  uint2 rsv = {0u, 0u};
  if (rows_ok) rsv = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(T.rscales) + rt * 16u + 4u * kg);
  // the lane's scale dword of each pass (token pass * 4 QP + d / 8, block 8 ct + d % 8 for
  // d = 64 wave + lane; past the pass's tokens: out of the buffer's range, zero)
  const __amdgpu_buffer_rsrc_t xs_r = buffer_rsrc(A.xs, 0x7FFFFFF0u);
  uint32_t xs_off[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const uint32_t d = 64u * wv + lane, jj = (uint32_t)p * 4u * QP + d / 8u;
    xs_off[p] = (d < 32u * QP && jj < ntok) ? ((tok ? tok[jj] : jj) * nkb + d % 8u) * 4u : 0x7FFFFFF0u;
  }
  build_lut<kW8KC, kW8T, 8, true>(lut_s, cbv, tid);

  float out[NQ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int v = 0; v < 4; ++v) out[q][v] = 0.f;

  // a pass's LDS: QP token rows per wave (1 KiB each, one direct-to-LDS load instruction; a row past
  // the tile's tokens reads nothing and writes zeros) and one scale instruction per wave
  auto stage = [&](int p, uint32_t ct) {
#pragma unroll
    for (int i = 0; i < QP; ++i) {
      const uint32_t jl = wv + 4u * (uint32_t)i, j = (uint32_t)p * 4u * QP + jl;
      const bool ok = j < ntok;
      const uint32_t t = ok ? (tok ? tok[j] : j) : 0u;
      const __amdgpu_buffer_rsrc_t r = buffer_rsrc(A.x8 + (uint64_t)t * A.cols + (uint64_t)ct * kTileCols, ok ? kTileCols : 0u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, AFFX_LDS_PTR(xb + jl * kW8Row), 16, lane * 16u, 0, 0, 0);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xs_r, AFFX_LDS_PTR(xsl + 64u * wv), 4, xs_off[p] + ct * 32u, 0, 0, 0);
  };

  for (uint32_t ct = 0; ct < nct; ++ct) {
    // this wave's unit of the column tile first (loads complete in issue order)
    Unit u;
    load_unit_ordered(u, codes, fields, (uint64_t)(rows_ok ? rt : 0u) * nct + ct, lane);
    v8i a[8];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      __syncthreads();  // the previous pass's reads of the LDS are done
      stage(p, ct);
      if (p == 0) {
        // the wave tile's eight A fragments, while the pass's rows arrive
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          uint32_t raw[8], bv[2];
          pin_step(u, m);
          lut_lookup_step<kW8KC, true>(u, lut, nullptr, copy4, m, raw, bv);
          a[m] = lut_finish(raw, bv);
          asm volatile("" ::: "memory");  // one step's table reads in flight at a time (registers)
        }
      }
      __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(0));
      __syncthreads();
      if (!rows_ok) continue;
#pragma unroll
      for (int ql = 0; ql < QP; ++ql) {
        const int q = p * QP + ql;
        const uint32_t jl = 4u * (uint32_t)ql + (c >> 2);
        const bool live = (c & 3u) == kg && (uint32_t)p * 4u * QP + jl < ntok;
        const uint8_t* bsrc = xb + jl * kW8Row + kg * (uint32_t)kSegCols;
        v4f acc0 = v4f{0.f, 0.f, 0.f, 0.f}, acc1 = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          v8i b = v8i{0, 0, 0, 0, 0, 0, 0, 0};
          if (live) b = b_step(reinterpret_cast<const u32x4*>(bsrc), m);
          if (m < 4)
            acc0 = mfma(a[m], b, acc0);
          else
            acc1 = mfma(a[m], b, acc1);
        }
        // the token's scales of the tile's eight blocks
        const float4 s0 = *reinterpret_cast<const float4*>(xsl + jl * 8u);
        const float4 s1 = *reinterpret_cast<const float4*>(xsl + jl * 8u + 4u);
        const float sb[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        // block 2g + h of the tile: group g's partial (lane g of the quad, a DPP quad broadcast), half h
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float o = out[q][v];
          o = __builtin_fmaf(quad_lane<0>(acc0[v]), sb[0], o);
          o = __builtin_fmaf(quad_lane<0>(acc1[v]), sb[1], o);
          o = __builtin_fmaf(quad_lane<1>(acc0[v]), sb[2], o);
          o = __builtin_fmaf(quad_lane<1>(acc1[v]), sb[3], o);
          o = __builtin_fmaf(quad_lane<2>(acc0[v]), sb[4], o);
          o = __builtin_fmaf(quad_lane<2>(acc1[v]), sb[5], o);
          o = __builtin_fmaf(quad_lane<3>(acc0[v]), sb[6], o);
          o = __builtin_fmaf(quad_lane<3>(acc1[v]), sb[7], o);
          out[q][v] = o;
        }
        // one quad at a time: the next quad's B reads are not hoisted over this one's MFMAs (a
        // compiler memory barrier; the registers of every quad's operands at once would cut the
        // waves a SIMD holds to one)
#pragma unroll
        for (int v = 0; v < 4; ++v) AFFX_PIN(out[q][v]);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  if (!rows_ok || (c & 3u) != 0u) return;
  const float rs[4] = {__uint_as_float(rsv.x << 16) * A.wscale, __uint_as_float(rsv.x & 0xFFFF0000u) * A.wscale,
                       __uint_as_float(rsv.y << 16) * A.wscale, __uint_as_float(rsv.y & 0xFFFF0000u) * A.wscale};
  const uint32_t ld = T.ld ? T.ld : T.nt;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const uint32_t j = 4u * q + (c >> 2);
    if (j >= ntok) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint64_t at = (uint64_t)(rt * 16u + 4u * kg + v) * ld + j;
      const float val = out[q][v] * rs[v];
      if (A.y_bf16)
        reinterpret_cast<uint16_t*>(T.y)[at] = w8_bf16(val);
      else
        reinterpret_cast<float*>(T.y)[at] = val;
    }
  }
}

}  // namespace affx

using namespace affx;

namespace {

template <int NQ>
int w8a8_launch(const W8a8Args& A, uint32_t n_tiles, hipStream_t s) {
  constexpr int NP = (4 * NQ + (int)kW8Pass - 1) / (int)kW8Pass, QP = NQ / NP;
  const uint32_t lds = 4u * QP * kW8Row + 4u * 64u * 4u;
  int rc = check_hip(hipFuncSetAttribute((const void*)w8a8_gemm_kernel<NQ>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)lds),
                     "hipFuncSetAttribute(w8a8)");
  if (rc) return rc;
  const dim3 g((A.rows / kTileRows + kW8Waves - 1) / kW8Waves * n_tiles);
  hipLaunchKernelGGL((w8a8_gemm_kernel<NQ>), g, dim3(kW8T), lds, s, A);
  return check_launch("w8a8_gemm_kernel");
}

}  // namespace

extern "C" int affx_expert_gemm_w8a8(const affx_expert_tile* tiles, uint32_t n_tiles, uint32_t max_nt, const void* x8,
                                     const float* xs, const uint32_t* codebook, uint32_t rows, uint32_t cols,
                                     float wscale, int y_bf16, void* stream) {
  if (n_tiles == 0) return AFFX_OK;
  if (!tiles || !x8 || !xs || !codebook) return set_error(AFFX_ERR_ARG, "expert_gemm_w8a8: null pointer");
  if (rows == 0 || rows % kTileRows || cols == 0 || cols % kTileCols || max_nt == 0 || max_nt > kW8MaxTok ||
      n_tiles > 65535u || (uint64_t)rows * cols > 0xFFFFFFFFull)
    return set_error(AFFX_DECLINED, "expert_gemm_w8a8: needs rows %% 16 == 0, cols a multiple of 1024, 1 <= max_nt "
                     "<= %u and at most 65535 tiles (got %u x %u, max_nt %u, %u tiles)", kW8MaxTok, rows, cols,
                     max_nt, n_tiles);
  if ((reinterpret_cast<uintptr_t>(x8) | reinterpret_cast<uintptr_t>(xs)) & 15u)
    return set_error(AFFX_ERR_ARG, "expert_gemm_w8a8: x8 and xs must be 16-byte aligned");
  W8a8Args A;
  A.tiles = tiles;
  A.x8 = (const uint8_t*)x8;
  A.xs = xs;
  A.codebook = codebook;
  A.rows = rows;
  A.cols = cols;
  A.wscale = wscale;
  A.y_bf16 = y_bf16 ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  const uint32_t nq = (max_nt + 3u) / 4u;
  if (nq <= 1) return w8a8_launch<1>(A, n_tiles, s);
  if (nq <= 2) return w8a8_launch<2>(A, n_tiles, s);
  if (nq <= 4) return w8a8_launch<4>(A, n_tiles, s);
  if (nq <= 8) return w8a8_launch<8>(A, n_tiles, s);
  return w8a8_launch<16>(A, n_tiles, s);
}
