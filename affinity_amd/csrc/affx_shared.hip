// The step after the routed experts, on the device: the shared expert (a dense FP8 SwiGLU FFN that
// every token runs, added into the block the routed experts wrote) and the hyper-connection post
// (the block folded into the residual lanes, leaving the block zero for the next sublayer).
//
// The shared expert's weights are the checkpoint's FP8 values (src/engine/matvec_fp8.inc:1-16):
// E4M3 bytes and one UE8M0 scale per 128x128 tile, the bytes permuted once at upload into a tile
// layout (below) so that each load instruction of a wave reads 1 KiB contiguous. They go to the
// fp8 MFMA as they are: a lane's A operand is 32 weight bytes of one row straight from memory, and
// the tile scale is the MFMA's own A scale (a lane's scale covers its 32 K values of one row,
// which never straddle a 128-column tile). The activations are E4M3 terms as on the
// routed path (t0 + t1/16 + t2/256 in adjacent B columns); their exponent is the B scale where it
// is one per wave (decode, and the batch down), else applied in the epilogue.
//
// Decode, 1..8 tokens (DenseOps::shexp, src/engine/model.h:314-319; the reference's device form
// mv_gate_up_swiglu_hip + launch_mv, src/gpu/dense_gpu.hip:2030-2116), two launches:
//   shexp_gateup     one workgroup per 8 rows of inter; 8 waves = {gate, up} x 4 K quarters, every
//                    weight load issued at the start; meanwhile the workgroup turns x into three
//                    E4M3 terms per element in LDS (one exponent per token); fixed-order sum of the
//                    quarters, SwiGLU with the clamp, three E4M3 terms out
//   shexp_down       one workgroup per 16 rows of hidden; 8 waves = 8 K eighths; fixed-order sum,
//                    y (+)= result
// Batch (BatchOps::shexp, src/engine/model.h:504-505; DenseGpu::batch_shexp, src/gpu/dense_gpu.hip:
// 4897-4950):
//   shexp_prep_rows  per token: exponent and 2 or 3 E4M3 terms of the bf16 row (+ low part)
//   shexp_gemm<0>    (128 rows of inter, token tile): gate and up, SwiGLU, terms out
//   shexp_gemm<1>    (256 rows of hidden, token tile): down, y (+)= result
// The hyper-connection post: DenseGpu::hc_post (src/gpu/dense_gpu.hip:2394-2465, kernels
// 1674-1724) and batch_hc_post (4517-4534, kernels src/gpu/batch_kernels.hip:1977-2019).
#include <cstdlib>
#include <cstring>

#include "affx_lut.h"

namespace affx {

struct SharedArgs {
  const uint8_t* w[3];  // gate, up [inter x hidden], down [hidden x inter]: E4M3 row-major
  const uint8_t* s[3];  // their UE8M0 tile scales, [rows / 128][cols / 128]
  uint32_t hidden, inter, m_tokens;
  uint8_t* aq;             // [M][3][inter]: SwiGLU output terms, exponent sigma_a
  float limit;
  int32_t sigma_a;
  float* y;
  uint64_t y_ts, y_ds;
  int accumulate;
};

constexpr int kSxWaves = 8;

// v8i from two 16-byte halves
__device__ __forceinline__ v8i join8(u32x4 lo, u32x4 hi) {
  v8i v;
  v[0] = (int)lo[0]; v[1] = (int)lo[1]; v[2] = (int)lo[2]; v[3] = (int)lo[3];
  v[4] = (int)hi[0]; v[5] = (int)hi[1]; v[6] = (int)hi[2]; v[7] = (int)hi[3];
  return v;
}

__device__ __forceinline__ v4f mfma_scaled(v8i a, v8i b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

// SwiGLU with the reference's asymmetric clamp (src/engine/ops.cpp:47-60); the clamp limit is > 0
// here (the entries decline a non-positive one).
__device__ __forceinline__ float swiglu_clamped(float g, float u, float L) {
  g = (L < g) ? L : g;
  const float lo = (-L < u) ? u : -L;
  u = (lo < L) ? lo : L;
  return (g / (1.0f + expf(-g))) * u;
}

// ------------------------------------------------------------------------------------------------
// device layout of a dense FP8 matrix
// ------------------------------------------------------------------------------------------------
// [rows x cols] (rows % 16 == 0, cols % 128 == 0) in 2 KiB chunks, one per 16-row tile rt
// (row-tile major) and 128-column step m: [half h][lane][16 B], lane = c + 16 kg holding row
// 16 rt + c, columns 128 m + 64 h + 16 kg .. + 15. One 16-byte load per lane then reads 1 KiB
// contiguous, already in the K order of the scaled fp8 MFMA used here (lane group kg holds the
// step's columns 16 kg + [0, 16) and 64 + 16 kg + [0, 16)).
__host__ __device__ inline uint32_t dense_tile_offset(uint32_t rt, uint32_t m, uint32_t cols) {
  return (rt * (cols >> 7) + m) * 2048u;
}

__global__ void __launch_bounds__(256) dense_fp8_permute_kernel(const uint8_t* __restrict__ src,
                                                                uint8_t* __restrict__ dst, uint32_t rows,
                                                                uint32_t cols) {
  const uint64_t q = (uint64_t)blockIdx.x * 256u + threadIdx.x;  // 16-byte chunk of dst
  if (q >= (uint64_t)rows * cols / 16u) return;
  const uint32_t lane = (uint32_t)(q & 63u), h = (uint32_t)((q >> 6) & 1u);
  const uint32_t tm = (uint32_t)(q >> 7), steps = cols >> 7, rt = tm / steps, m = tm % steps;
  const uint32_t r = 16u * rt + (lane & 15u), k = 128u * m + 64u * h + 16u * (lane >> 4);
  *reinterpret_cast<uint4*>(dst + 16u * q) = *reinterpret_cast<const uint4*>(src + (uint64_t)r * cols + k);
}

// ------------------------------------------------------------------------------------------------
// decode
// ------------------------------------------------------------------------------------------------
// K order inside a 128-column MFMA step: lane group kg holds columns 16 kg .. 16 kg + 15 and
// 64 + 16 kg .. 64 + 16 kg + 15 (any order works as long as A and B agree), so each of a step's two
// 16-byte weight loads reads 64 contiguous bytes of each of the tile's 16 rows.

// The weights of one wave's share of a 16-row tile, all requested at once: rows row0 .. row0 + 15
// of W [.. x K], columns k0 .. k0 + 128 STEPS - 1; sa[m] = the tile scale of step m (the rows lie
// in one 128-row band: uniform). half >= 0: only rows row0 + 8 half .. + 7 are read, the others'
// A rows are zero. The scales are requested before the weights: loads complete in issue order, so
// their readfirstlane waits for them alone, not for the weights behind them (issued after the
// weights, it made the whole wave wait for every weight before its activation work).
template <int STEPS>
__device__ __forceinline__ void load_a_tile(const uint8_t* __restrict__ W, const uint8_t* __restrict__ S, uint32_t K,
                                            uint32_t row0, uint32_t k0, v8i (&a)[STEPS], int (&sa)[STEPS],
                                            int half = -1) {
  const uint32_t lane = threadIdx.x & 63, c = lane & 15, kg = lane >> 4;
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), (short)0, 0x7FFFFFFF, 0x00020000);
  // lanes outside the half take an offset past the buffer's range: the load returns zero and
  // touches no memory, with no branch around it (a branch made the compiler wait for every load
  // at its join)
  const bool mine = half < 0 || (int)(c >> 3) == half;
  const uint32_t vo = mine ? dense_tile_offset(row0 >> 4, k0 >> 7, K) + 16u * lane : 0x80000000u;
  // (one byte load each: byte reads of an ordinary pointer are merged into one wide load whose
  // byte extraction then waits for it before the weights are requested)
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(S), (short)0, 0x7FFFFFFF, 0x00020000);
  const uint32_t so = (row0 >> 7) * (K >> 7) + (k0 >> 7);
  int sv[STEPS];
#pragma unroll
  for (int m = 0; m < STEPS; ++m) sv[m] = (int)__builtin_amdgcn_raw_buffer_load_b8(sr, so + (uint32_t)m, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < STEPS; ++m)
    a[m] = join8(__builtin_amdgcn_raw_buffer_load_b128(wr, vo + 2048u * m, 0, 2),
                 __builtin_amdgcn_raw_buffer_load_b128(wr, vo + 2048u * m + 1024u, 0, 2));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < STEPS; ++m) sa[m] = __builtin_amdgcn_readfirstlane(sv[m]);
}

// Column c of B column group cg: token 5 cg + c / 3, term c % 3 (column 15 unused).
__device__ __forceinline__ uint32_t bcol_token(int cg, uint32_t c) { return 5u * cg + c / 3u; }

// The three E4M3 terms of token t held in columns c, c + 1, c + 2 of a 16-column group.
__device__ __forceinline__ float part_terms(const float (&p)[16], uint32_t col) {
  return p[col] + p[col + 1] * 0.0625f + p[col + 2] * 0.00390625f;
}

// gate/up + SwiGLU: one workgroup per 8 rows of inter (half of a 16-row tile: twice the
// workgroups of one per tile, so every CU streams weights; the MFMA rows of the other half are
// zero), wave w = {gate, up}[w & 1] x K quarter w >> 1 (STEPS = hidden / 512 steps each). The
// activation's terms are made here, into LDS: each thread holds 8 columns of every token, the
// token's largest magnitude fixes its exponent (the B scale), three E4M3 terms per element.
template <int CG, int STEPS, bool VEC, int TOK>
__global__ void __launch_bounds__(kSxWaves * 64) shexp_gateup_kernel(SharedArgs A, const float* __restrict__ x,
                                                                     uint64_t xts, uint64_t xds) {
  const uint32_t rt = blockIdx.x >> 1, half = blockIdx.x & 1u, tid = threadIdx.x, lane = tid & 63;
  // the wave index in a scalar register: the weight and scale pointers it selects stay scalar (a
  // vector index made the compiler fetch them with vector loads and wrap every weight load in a
  // loop over the distinct buffer descriptors)
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t c = lane & 15, kg = lane >> 4;
  const uint32_t mat = wv & 1u, q = wv >> 1, M = A.m_tokens, H = A.hidden;
  const uint32_t k0 = q * (H / 4u);
  __shared__ __align__(16) uint8_t xq_l[TOK * kTerms * 4096];
  __shared__ float part[kSxWaves][CG][16][16];
  __shared__ float red[kSxWaves][kMaxTok];
  // 1. the activation (small, in the cache) first: loads complete in issue order, so the wait for
  // it does not wait for the weights issued after it. The loads are unconditional (tokens past M
  // and columns past H read token 0 and column 0, and are zeroed at their use): a load under a
  // branch made the compiler wait for it at the join, before the weights were requested. TOK is
  // the most tokens the launch holds (1 for batch 1: every workgroup reads the whole activation,
  // so padding tokens would multiply that traffic).
  static_assert(TOK <= 5 * CG && TOK <= kMaxTok, "");
  const uint32_t h0 = 8u * tid;
  const bool mine = h0 < H;
  const uint32_t hl = mine ? h0 : 0u;
  float xv[kMaxTok][8];
#pragma unroll
  for (int t = 0; t < kMaxTok; ++t) {
    const uint64_t tt = (uint32_t)t < M ? (uint32_t)t : 0u;
    if (t >= TOK) {
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[t][i] = 0.f;
    } else if constexpr (VEC) {  // token-major rows, 16-byte aligned
      const float4 v0 = *reinterpret_cast<const float4*>(x + tt * xts + hl);
      const float4 v1 = *reinterpret_cast<const float4*>(x + tt * xts + hl + 4);
      xv[t][0] = v0.x; xv[t][1] = v0.y; xv[t][2] = v0.z; xv[t][3] = v0.w;
      xv[t][4] = v1.x; xv[t][5] = v1.y; xv[t][6] = v1.z; xv[t][7] = v1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[t][i] = x[tt * xts + (hl + i) * xds];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. the weights
  v8i a[STEPS];
  int sa[STEPS];
  load_a_tile<STEPS>(A.w[mat], A.s[mat], H, rt * 16u, k0, a, sa, (int)half);
  __builtin_amdgcn_sched_barrier(0);
  // 3. exponent per token: its largest magnitude times 2^sigma in [128, 256)
#pragma unroll
  for (int t = 0; t < TOK; ++t)
    if (!((uint32_t)t < M && mine))
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[t][i] = 0.f;
#pragma unroll
  for (int t = 0; t < TOK; ++t) {
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(xv[t][i]));
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) red[wv][t] = mx;
  }
  __syncthreads();
  int sig[kMaxTok];
#pragma unroll
  for (int t = 0; t < kMaxTok; ++t) {
    float mx = 0.f;
    if (t < TOK)
#pragma unroll
      for (int w = 0; w < kSxWaves; ++w) mx = fmaxf(mx, red[w][t]);
    sig[t] = mx > 0.f ? 7 - ilogbf(mx) : 0;
  }
  // 4. three E4M3 terms of every element into LDS, [token][term][column]
#pragma unroll
  for (int t = 0; t < kMaxTok; ++t)
    if ((uint32_t)t < M && mine) {
      uint32_t p0, p1, p2, q0, q1, q2;
      split3x4(ldexpf(xv[t][0], sig[t]), ldexpf(xv[t][1], sig[t]), ldexpf(xv[t][2], sig[t]), ldexpf(xv[t][3], sig[t]),
               p0, p1, p2);
      split3x4(ldexpf(xv[t][4], sig[t]), ldexpf(xv[t][5], sig[t]), ldexpf(xv[t][6], sig[t]), ldexpf(xv[t][7], sig[t]),
               q0, q1, q2);
      uint8_t* dst = xq_l + (uint32_t)t * kTerms * H + h0;
      *reinterpret_cast<uint2*>(dst) = uint2{p0, q0};
      *reinterpret_cast<uint2*>(dst + H) = uint2{p1, q1};
      *reinterpret_cast<uint2*>(dst + 2 * H) = uint2{p2, q2};
    }
  __syncthreads();
  // 5. one MFMA per step and column group, B from LDS
  v4f acc[CG];
  int sb[CG];
  const uint8_t* bp[CG];
  bool bv[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const uint32_t t = bcol_token(cg, c);
    bv[cg] = c < 15u && t < M;
    bp[cg] = xq_l + (bv[cg] ? (t * kTerms + c % 3u) * H : 0u) + k0 + 16u * kg;
    sb[cg] = 127 - (bv[cg] ? sig[t < (uint32_t)kMaxTok ? t : 0] : 0);
    acc[cg] = v4f{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int m = 0; m < STEPS; ++m)
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      v8i b = join8(*reinterpret_cast<const u32x4*>(bp[cg] + 128 * m), *reinterpret_cast<const u32x4*>(bp[cg] + 128 * m + 64));
      if (!bv[cg]) b = v8i{0, 0, 0, 0, 0, 0, 0, 0};
      acc[cg] = mfma_scaled(a[m], b, acc[cg], sa[m], sb[cg]);
    }
  // accumulator lane l, element v = D[row 4 (l / 16) + v][column l % 16]
#pragma unroll
  for (int cg = 0; cg < CG; ++cg)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wv][cg][4 * kg + v][c] = acc[cg][v];
  __syncthreads();
  if (tid < 16u * M && ((tid & 15u) >> 3) == half) {
    const uint32_t r = tid & 15u, t = tid >> 4, cg = t / 5u, col = (t % 5u) * 3u;
    float g = 0.f, u = 0.f;
    for (uint32_t qq = 0; qq < 4; ++qq) {  // K quarters in order
      g += part_terms(part[2 * qq][cg][r], col);
      u += part_terms(part[2 * qq + 1][cg][r], col);
    }
    const float a = swiglu_clamped(g, u, A.limit);
    uint32_t b0, b1, b2;
    split3(ldexpf(a, A.sigma_a), b0, b1, b2);
    uint8_t* dst = A.aq + (uint64_t)t * kTerms * A.inter + rt * 16u + r;
    dst[0] = (uint8_t)b0;
    dst[A.inter] = (uint8_t)b1;
    dst[2 * (uint64_t)A.inter] = (uint8_t)b2;
  }
}

// down: one workgroup per 16 rows of hidden, wave w = K eighth w (STEPS = inter / 1024 steps); B
// (the SwiGLU terms, small, in the cache) requested before the weights; fixed-order sum of the
// eighths; y (+)= result.
template <int CG, int STEPS>
__global__ void __launch_bounds__(kSxWaves * 64) shexp_down_kernel(SharedArgs A) {
  const uint32_t rt = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, M = A.m_tokens;
  const uint32_t c = lane & 15, kg = lane >> 4;
  const uint32_t k0 = wv * (A.inter / 8u);
  __shared__ float part[kSxWaves][CG][16][16];
  v8i b[STEPS][CG];
  // columns without a token read past the buffer's range (zero, no memory touched): a select on
  // the loaded values would make the wave wait for them before it requests the weights
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(A.aq, (short)0, 0x7FFFFFFF, 0x00020000);
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const uint32_t t = bcol_token(cg, c);
    const bool ok = c < 15u && t < M;
    const uint32_t bo = ok ? (t * kTerms + c % 3u) * A.inter + k0 + 16u * kg : 0x80000000u;
#pragma unroll
    for (int m = 0; m < STEPS; ++m)
      b[m][cg] = join8(__builtin_amdgcn_raw_buffer_load_b128(br, bo + 128u * m, 0, 0),
                       __builtin_amdgcn_raw_buffer_load_b128(br, bo + 128u * m + 64u, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  v8i a[STEPS];
  int sa[STEPS];
  load_a_tile<STEPS>(A.w[2], A.s[2], A.inter, rt * 16u, k0, a, sa);
  const int sb = 127 - A.sigma_a;
  v4f acc[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) acc[cg] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < STEPS; ++m)
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) acc[cg] = mfma_scaled(a[m], b[m][cg], acc[cg], sa[m], sb);
#pragma unroll
  for (int cg = 0; cg < CG; ++cg)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wv][cg][4 * kg + v][c] = acc[cg][v];
  __syncthreads();
  if (tid < 16u * M) {
    const uint32_t r = tid & 15u, t = tid >> 4, cg = t / 5u, col = (t % 5u) * 3u;
    float sum = 0.f;
    for (uint32_t qq = 0; qq < (uint32_t)kSxWaves; ++qq) sum += part_terms(part[qq][cg][r], col);  // in order
    float* yp = A.y + t * A.y_ts + (uint64_t)(rt * 16u + r) * A.y_ds;
    *yp = A.accumulate ? *yp + sum : sum;
  }
}

// ------------------------------------------------------------------------------------------------
// batch: a dense fp8 GEMM over token tiles
// ------------------------------------------------------------------------------------------------
// One workgroup = one (row block, token tile), 8 waves, each 32 weight rows (two 16-row tiles:
// gate/up = 16 rows of gate and the same rows of up, down = two tiles) against the tile's 192 B
// columns (12 MFMA column tiles; a token is TX adjacent columns, 16 / TX tokens per column tile).
// Per 128-column MFMA step: the wave's weights come straight from memory into registers, two
// steps ahead; the B columns come into LDS by direct loads, two steps ahead in four buffers (one
// workgroup barrier per two steps), 16-byte chunks swizzled by column so the fragment reads of 16
// lanes hit 16 distinct bank groups. Items map to XCDs by row block: workgroup i runs on XCD i % 8,
// and all token tiles of a row block run on one XCD, whose L2 then holds that block's weights.
constexpr int kBW = 8;
constexpr int kBT = kBW * 64;
constexpr int kBRT = 2;
constexpr int kBCT = 12;
constexpr int kBCols = kBCT * 16;
constexpr uint32_t kBBuf = kBCols * 128;
constexpr int kBDma = kBCols / 8 / kBW;

struct SharedGemmArgs {
  const uint8_t* w0;  // gate (PH 0) or down (PH 1)
  const uint8_t* s0;
  const uint8_t* w1;  // up (PH 0)
  const uint8_t* s1;
  uint32_t K;         // columns of the weights
  uint32_t n_tok, n_tiles, n_rb;
  const uint8_t* ws;  // B rows at ws + b_off + (token * TX + term) * K; a zero row at ws + zero_off
  uint64_t b_off, zero_off;
  const int32_t* sigma;  // per token: exponent of its x terms (PH 0)
  int32_t sigma_a;       // exponent of the SwiGLU terms
  uint32_t inter, hidden;
  uint8_t* aq;           // PH 0 output [token][3][inter]
  float* y;              // PH 1 output [token][hidden]
  int accumulate;
  float limit;
};

template <int PH, int TX>
__global__ void __launch_bounds__(kBT, 1) shexp_gemm_kernel(SharedGemmArgs A) {
  constexpr int TPG = 16 / TX;       // tokens per 16-column tile
  constexpr int TT = kBCT * TPG;     // tokens per workgroup tile
  const uint32_t i = blockIdx.x, l = i >> 3;
  const uint32_t rb = (i & 7u) + 8u * (l / A.n_tiles), tile = l % A.n_tiles;
  if (rb >= A.n_rb) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63, c = lane & 15, kg = lane >> 4;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t K = A.K, nsteps = K / 128u, tok0 = tile * TT;

  __shared__ __align__(16) uint8_t buf0[kBBuf];
  __shared__ __align__(16) uint8_t buf1[kBBuf];
  __shared__ __align__(16) uint8_t buf2[kBBuf];
  __shared__ __align__(16) uint8_t buf3[kBBuf];
  uint32_t* rowoff = reinterpret_cast<uint32_t*>(buf3);  // set-up only, before buffer 3 is written
  auto bufsel = [&](int b) -> uint8_t* { return b == 0 ? buf0 : b == 1 ? buf1 : b == 2 ? buf2 : buf3; };

  // the wave's row tiles: gate/up = rows rb*128 + 16 wv of gate (r = 0) and of up (r = 1); down =
  // rows rb*256 + 32 wv + 16 r
  const uint32_t rowt = PH == 0 ? rb * 128u + 16u * wv : rb * 256u + 32u * wv;
  auto row_of = [&](int r) -> uint32_t { return PH == 0 ? rowt : rowt + 16u * r; };
  const __amdgpu_buffer_rsrc_t wr0 =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(A.w0), (short)0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr1 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(PH == 0 ? A.w1 : A.w0), (short)0, 0x7FFFFFFF, 0x00020000);
  uint32_t vo[kBRT];
#pragma unroll
  for (int r = 0; r < kBRT; ++r) vo[r] = dense_tile_offset(row_of(r) >> 4, 0, K) + 16u * lane;
  v8i ring[4][kBRT];
  auto a_load = [&](int slot, uint32_t t) {
#pragma unroll
    for (int r = 0; r < kBRT; ++r) {
      const __amdgpu_buffer_rsrc_t wr = r == 0 ? wr0 : wr1;
      ring[slot][r] = join8(__builtin_amdgcn_raw_buffer_load_b128(wr, vo[r] + 2048u * t, 0, 2),
                            __builtin_amdgcn_raw_buffer_load_b128(wr, vo[r] + 2048u * t + 1024u, 0, 2));
    }
  };
  // scale rows of the two tiles (a 128-row band each), one dword = four steps
  const uint8_t* srow0 = A.s0 + (uint64_t)(row_of(0) >> 7) * (K >> 7);
  const uint8_t* srow1 = (PH == 0 ? A.s1 : A.s0) + (uint64_t)(row_of(1) >> 7) * (K >> 7);

  // B column j of the tile: token tok0 + (j / 16) TPG + (j % 16) / TX, term (j % 16) % TX
  auto col_token = [&](uint32_t j, bool& used) -> uint32_t {
    const uint32_t cc = j & 15u, tok = tok0 + (j >> 4) * TPG + cc / TX;
    used = cc < (uint32_t)(TX * TPG) && tok < A.n_tok;
    return tok;
  };
  if (tid < (uint32_t)kBCols) {
    bool used;
    const uint32_t tok = col_token(tid, used);
    rowoff[tid] = used ? (uint32_t)(A.b_off + ((uint64_t)tok * TX + (tid & 15u) % TX) * K) : (uint32_t)A.zero_off;
  }
  // B scale: the SwiGLU terms' exponent for down; gate/up applies each token's own exponent in
  // the epilogue (a per-lane scale for each column tile would cost twelve registers)
  const int sbu = PH == 0 ? 127 : 127 - A.sigma_a;
  __syncthreads();
  // DMA lane map: instruction i of wave w writes columns 8b .. 8b + 7 (b = kBDma w + i), lane l to
  // LDS slot l & 7 of column 8b + (l >> 3); slot p of column col holds global chunk p ^ f(col),
  // f(col) = (cc ^ (cc >> 3)) & 7 with cc = col & 15
  uint32_t roff[kBDma];
#pragma unroll
  for (int d = 0; d < kBDma; ++d) {
    const uint32_t col = 8u * (kBDma * wv + d) + (lane >> 3);
    const uint32_t cc = col & 15u;
    roff[d] = rowoff[col] + ((((lane & 7u) ^ ((cc ^ (cc >> 3)) & 7u))) << 4);
  }
  const __amdgpu_buffer_rsrc_t wsr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(A.ws), (short)0, (int)0xFFFFFFFF, 0x00020000);
  auto dma = [&](uint8_t* b, uint32_t t) {
#pragma unroll
    for (int d = 0; d < kBDma; ++d)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, AFFX_LDS_PTR(b + (kBDma * wv + d) * 1024u), 16, roff[d],
                                               t * 128u, 0, 0);
  };
  // the lane's two 16-byte chunks of a step in the MFMA K order (kg and 4 + kg; the swizzle keeps
  // the 16 lanes of each K group on 16 distinct bank groups)
  const uint32_t bo0 = c * 128u + (((kg) ^ ((c ^ (c >> 3)) & 7u)) << 4);
  const uint32_t bo1 = c * 128u + (((4u + kg) ^ ((c ^ (c >> 3)) & 7u)) << 4);
  auto bread = [&](const uint8_t* b, int ct) -> v8i {
    return join8(*reinterpret_cast<const u32x4*>(b + ct * 2048 + bo0),
                 *reinterpret_cast<const u32x4*>(b + ct * 2048 + bo1));
  };

  // set-up: B of steps 0 and 1, weights of steps 0 and 1; rowoff (in buffer 3) is read before
  // any wave writes buffer 3 (step 0, after the barrier below)
  __syncthreads();
  dma(buf0, 0);
  dma(buf1, 1);
  __builtin_amdgcn_sched_barrier(0);
  a_load(0, 0);
  a_load(1, 1);
  __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(4 * kBRT));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  v4f acc[kBRT][kBCT];
#pragma unroll
  for (int r = 0; r < kBRT; ++r)
#pragma unroll
    for (int ct = 0; ct < kBCT; ++ct) acc[r][ct] = v4f{0.f, 0.f, 0.f, 0.f};

  // step t = 4 g + m: B in buffer m, weights in ring slot m. Loads past the last step repeat the
  // last step's (their data is not used), so the count of loads in flight is the same on every
  // path and the wait counts below are constants.
  for (uint32_t g = 0; g < nsteps / 4u; ++g) {
    const uint32_t sc0 = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t*>(srow0 + 4u * g));
    const uint32_t sc1 = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t*>(srow1 + 4u * g));
    static_for<0, 4>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      const uint32_t t = 4u * g + m;
      if constexpr ((m & 1) == 0) {
        const uint32_t t2 = t + 2u < nsteps ? t + 2u : nsteps - 1u, t3 = t + 3u < nsteps ? t + 3u : nsteps - 1u;
        dma(bufsel((m + 2) & 3), t2);
        dma(bufsel((m + 3) & 3), t3);
      }
      __builtin_amdgcn_sched_barrier(0);
      a_load((m + 2) & 3, t + 2u < nsteps ? t + 2u : nsteps - 1u);
      __builtin_amdgcn_sched_barrier(0);
      // this step's weights were issued two steps ago; after them came two steps of weights (two
      // loads per tile each: 4 kBRT) and one pair of B steps (2 kBDma)
      __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(4 * kBRT + 2 * kBDma));
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* bcur = bufsel(m);
      static_for<0, kBCT>([&](auto cc) {
        constexpr int ct = decltype(cc)::value;
        const v8i bq = bread(bcur, ct);
        acc[0][ct] = mfma_scaled(ring[m][0], bq, acc[0][ct], (int)((sc0 >> (8 * m)) & 0xFFu), sbu);
        acc[1][ct] = mfma_scaled(ring[m][1], bq, acc[1][ct], (int)((sc1 >> (8 * m)) & 0xFFu), sbu);
      });
      // after an odd step t the B of steps t + 1 and t + 2 (issued at the top of step t - 1) has
      // landed once at most the weights issued after it (steps t - 1 and t) are outstanding
      if constexpr ((m & 1) == 1) {
        __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(4 * kBRT));
        __builtin_amdgcn_s_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  }
  __builtin_amdgcn_s_waitcnt(AFFX_VMCNT(0));

  // epilogue: accumulator lane (c, kg), element v = D[4 kg + v][c]; the lane whose column is a
  // token's first term combines the TX terms from its right neighbours
  auto terms = [&](float d) -> float {
    const float d1 = row_shl<1>(d);
    if constexpr (TX == 2) {
      return d + d1 * 0.0625f;
    } else {
      const float d2 = row_shl<2>(d);
      return d + d1 * 0.0625f + d2 * 0.00390625f;
    }
  };
  const float L = A.limit;
  static_for<0, kBCT>([&](auto cc) {
    constexpr int ct = decltype(cc)::value;
    bool used;
    const uint32_t tok = col_token(16u * ct + c, used);
    if constexpr (PH == 0) {
      float g4[4], u4[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        g4[v] = terms(acc[0][ct][v]);
        u4[v] = terms(acc[1][ct][v]);
      }
      if (used && c % TX == 0) {
        const int sig = A.sigma[tok];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          g4[v] = ldexpf(g4[v], -sig);
          u4[v] = ldexpf(u4[v], -sig);
        }
        float a[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float gv = g4[v], uv = u4[v];
          gv = (L < gv) ? L : gv;  // SwiGLU with the asymmetric clamp: src/engine/ops.cpp:47-60
          const float lo = (-L < uv) ? uv : -L;
          uv = (lo < L) ? lo : L;
          // (hardware exp2 and reciprocal: a few ulp, far inside the path's tolerance)
          const float e = __builtin_amdgcn_exp2f(-gv * 1.44269504f);
          a[v] = ldexpf(gv * __builtin_amdgcn_rcpf(1.0f + e) * uv, A.sigma_a);
        }
        uint32_t o0, o1, o2;
        split3x4(a[0], a[1], a[2], a[3], o0, o1, o2);
        uint8_t* dst = A.aq + (uint64_t)tok * 3 * A.inter + rowt + 4u * kg;
        *reinterpret_cast<uint32_t*>(dst) = o0;
        *reinterpret_cast<uint32_t*>(dst + A.inter) = o1;
        *reinterpret_cast<uint32_t*>(dst + 2 * (uint64_t)A.inter) = o2;
      }
    } else {
#pragma unroll
      for (int r = 0; r < kBRT; ++r) {
        float d4[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) d4[v] = terms(acc[r][ct][v]);
        if (used && c % TX == 0) {
          float4* yp = reinterpret_cast<float4*>(A.y + (uint64_t)tok * A.hidden + row_of(r) + 4u * kg);
          float4 o = A.accumulate ? *yp : make_float4(0.f, 0.f, 0.f, 0.f);
          o.x += d4[0];
          o.y += d4[1];
          o.z += d4[2];
          o.w += d4[3];
          *yp = o;
        }
      }
    }
  });
}

__global__ void __launch_bounds__(256) shexp_prep_rows_kernel(const uint16_t* __restrict__ x,
                                                              const uint16_t* __restrict__ xlo, uint32_t hidden,
                                                              uint32_t tx, int32_t* __restrict__ sigma,
                                                              uint8_t* __restrict__ xq, uint32_t* __restrict__ zeros,
                                                              uint32_t zero_words) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  if (t == 0)
    for (uint32_t i = tid; i < zero_words; i += 256) zeros[i] = 0u;
  __shared__ float red[4];
  const int s = row_terms<false>(x + (uint64_t)t * hidden, xlo ? xlo + (uint64_t)t * hidden : nullptr, hidden, tx,
                                 xq + (uint64_t)t * tx * hidden, red);
  if (tid == 0) sigma[t] = s;
}

// ------------------------------------------------------------------------------------------------
// hyper-connection post
// ------------------------------------------------------------------------------------------------
// Lane dst of the next state = block * post[dst] + sum over src in order of comb[dst + src NH] *
// lane src, each product rounded before its add exactly as the host's hc_expand
// (src/engine/ops.cpp:470-482) does it, so the result is the host's bit for bit. ZB: the block is
// the sublayer's accumulator and is left zero (the next sublayer accumulates into it).
template <uint32_t NH>
__global__ void __launch_bounds__(256) hc_expand_kernel(float* __restrict__ out_hc, float* __restrict__ block,
                                                        const float* __restrict__ hc, const float* __restrict__ post,
                                                        const float* __restrict__ comb, uint32_t n_embd, int zb) {
#pragma clang fp contract(off)
  const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= n_embd) return;
  const float b = block[d];
  float v[NH];
#pragma unroll
  for (uint32_t s = 0; s < NH; ++s) v[s] = hc[(uint64_t)s * n_embd + d];
#pragma unroll
  for (uint32_t dst = 0; dst < NH; ++dst) {
    float acc = b * post[dst];
#pragma unroll
    for (uint32_t s = 0; s < NH; ++s) acc += comb[dst + s * NH] * v[s];
    out_hc[(uint64_t)dst * n_embd + d] = acc;
  }
  if (zb) block[d] = 0.0f;
}

// A layer without a control: lane 0 += block (the block's length n).
__global__ void __launch_bounds__(256) hc_add_kernel(float* __restrict__ hc, float* __restrict__ block, uint64_t n,
                                                     int zb) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  hc[i] += block[i];
  if (zb) block[i] = 0.0f;
}

__device__ __forceinline__ uint16_t hc_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// The batch form over the engine's dim-major arenas (nb tokens): hc [NH][n_embd][nb] bf16, block
// [n_embd][nb] f32, post [NH][nb], comb [NH * NH][nb]; out [NH][n_embd][nb] bf16.
template <uint32_t NH>
__global__ void __launch_bounds__(256) hc_expand_batch_kernel(uint16_t* __restrict__ out_hc, float* __restrict__ block,
                                                              const uint16_t* __restrict__ hc,
                                                              const float* __restrict__ post,
                                                              const float* __restrict__ comb, uint32_t n_embd,
                                                              uint32_t nb, int zb) {
#pragma clang fp contract(off)
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t b = (uint32_t)(i % nb), d = (uint32_t)(i / nb);
  if (d >= n_embd) return;
  const float bv = block[i];
  float v[NH];
#pragma unroll
  for (uint32_t s = 0; s < NH; ++s) v[s] = __uint_as_float((uint32_t)hc[((uint64_t)s * n_embd + d) * nb + b] << 16);
#pragma unroll
  for (uint32_t dst = 0; dst < NH; ++dst) {
    float acc = bv * post[(uint64_t)dst * nb + b];
#pragma unroll
    for (uint32_t s = 0; s < NH; ++s) acc += comb[(uint64_t)(dst + s * NH) * nb + b] * v[s];
    out_hc[((uint64_t)dst * n_embd + d) * nb + b] = hc_bf16(acc);
  }
  if (zb) block[i] = 0.0f;
}

// Lane 0 of the bf16 batch state += block (n elements), rounded back to bf16.
__global__ void __launch_bounds__(256) hc_add_batch_kernel(uint16_t* __restrict__ hc, float* __restrict__ block,
                                                           uint64_t n, int zb) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  hc[i] = hc_bf16(__uint_as_float((uint32_t)hc[i] << 16) + block[i]);
  if (zb) block[i] = 0.0f;
}

// ------------------------------------------------------------------------------------------------
// batch, library-GEMM form
// ------------------------------------------------------------------------------------------------
// The weights widened to bf16 row-major, each value E4M3 x its tile's 2^(e - 127), exactly (an
// E4M3 value has at most four significant bits, and the product is a bf16 normal for tile exponents
// 10..254; below 10, scales under 2^-117 that no checkpoint holds, the product's low bits are cut;
// the exponent byte 255 and the E4M3 NaN codes give NaN). One launch for the three matrices, which
// have the same size; one thread per 16-byte piece of the tile layout (16 weights of one row): two
// hardware conversions per four bytes, the tile scale, the f32 product's high half (exact) packed,
// 32 bytes out, written `copies` times at column offsets 0 and copy_off of the output row.
struct WidenArgs {
  const uint8_t* w[3];
  const uint8_t* s[3];
  uint16_t* out[3];
  uint32_t rows[3], cols[3], ldo[3], copies[3], copy_off[3];
  uint32_t wg_per;  // workgroups per matrix
};

__global__ void __launch_bounds__(256) shexp_widen_kernel(WidenArgs W) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const uint32_t mi = blockIdx.x / W.wg_per;
  const uint32_t rows = W.rows[mi], cols = W.cols[mi];
  const uint64_t q = (uint64_t)(blockIdx.x - mi * W.wg_per) * 256u + threadIdx.x;
  if (mi >= 3u || q >= (uint64_t)rows * cols / 16u) return;
  const uint32_t steps = cols >> 7, chunk = (uint32_t)(q >> 7), lane = (uint32_t)q & 63u;
  const uint32_t half = ((uint32_t)q >> 6) & 1u, rt = chunk / steps, m = chunk - rt * steps;
  const uint32_t row = 16u * rt + (lane & 15u), col = 128u * m + 64u * half + 16u * (lane >> 4);
  const u32x4 v = *reinterpret_cast<const u32x4*>(W.w[mi] + q * 16u);
  const uint32_t e = W.s[mi][(uint64_t)(row >> 7) * steps + m];
  const float sc = e == 255u ? __uint_as_float(0x7FC00000u) : e ? __uint_as_float(e << 23) : __uint_as_float(0x00400000u);
  u32x4 o[2];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)v[d], false), hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)v[d], true);
    o[d >> 1][(d & 1) * 2] = __builtin_amdgcn_perm(__float_as_uint(lo[1] * sc), __float_as_uint(lo[0] * sc), 0x07060302u);
    o[d >> 1][(d & 1) * 2 + 1] = __builtin_amdgcn_perm(__float_as_uint(hi[1] * sc), __float_as_uint(hi[0] * sc), 0x07060302u);
  }
  uint16_t* p = W.out[mi] + (uint64_t)row * W.ldo[mi] + col;
  for (uint32_t c = 0; c < W.copies[mi]; ++c, p += W.copy_off[mi]) {
    reinterpret_cast<u32x4*>(p)[0] = o[0];
    reinterpret_cast<u32x4*>(p)[1] = o[1];
  }
}

// The SwiGLU between the two GEMMs: g [T][2 inter] f32 (gate columns, then up) -> a [T][2 inter]
// bf16, the output's high bf16 at column j and the rounded remainder at column inter + j (their
// sum carries 16 significant bits). Four columns a thread.
__global__ void __launch_bounds__(256) shexp_swiglu_split_kernel(const float* __restrict__ g, uint16_t* __restrict__ a,
                                                                 uint32_t inter, uint64_t quads, float limit) {
  const uint64_t q = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (q >= quads) return;
  const uint32_t per_row = inter >> 2;
  const uint64_t t = q / per_row;
  const uint32_t j = (uint32_t)(q - t * per_row) * 4u;
  const float* gr = g + t * 2u * inter;
  const float4 gv = *reinterpret_cast<const float4*>(gr + j), uv = *reinterpret_cast<const float4*>(gr + inter + j);
  const float r[4] = {swiglu_clamped(gv.x, uv.x, limit), swiglu_clamped(gv.y, uv.y, limit),
                      swiglu_clamped(gv.z, uv.z, limit), swiglu_clamped(gv.w, uv.w, limit)};
  uint32_t hi[2], lo[2];
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    const uint32_t h0 = hc_bf16(r[i]), h1 = hc_bf16(r[i + 1]);
    const uint32_t l0 = hc_bf16(r[i] - __uint_as_float(h0 << 16)), l1 = hc_bf16(r[i + 1] - __uint_as_float(h1 << 16));
    hi[i >> 1] = h0 | (h1 << 16);
    lo[i >> 1] = l0 | (l1 << 16);
  }
  uint16_t* ar = a + t * 2u * inter;
  *reinterpret_cast<uint64_t*>(ar + j) = (uint64_t)hi[0] | ((uint64_t)hi[1] << 32);
  *reinterpret_cast<uint64_t*>(ar + inter + j) = (uint64_t)lo[0] | ((uint64_t)lo[1] << 32);
}

}  // namespace affx

using namespace affx;

namespace {

struct SharedWs {
  uint64_t sigma, zeros, xq, aq, total;
};

// decode: [aq M x 3 x inter]
SharedWs shared_decode_ws(uint32_t M, uint32_t hidden, uint32_t inter) {
  (void)hidden;
  SharedWs w;
  w.sigma = w.zeros = w.xq = w.aq = 0;
  w.total = a256((uint64_t)M * kTerms * inter);
  return w;
}

// batch: [sigma T][zeros max(hidden, inter)][xq T x 3 x hidden][aq T x 3 x inter]
SharedWs shared_batch_ws(uint32_t T, uint32_t hidden, uint32_t inter) {
  SharedWs w;
  w.sigma = 0;
  w.zeros = a256(4ull * T);
  w.xq = w.zeros + a256(hidden > inter ? hidden : inter);
  w.aq = w.xq + a256((uint64_t)T * kTerms * hidden);
  w.total = w.aq + a256((uint64_t)T * kTerms * inter);
  return w;
}

// batch, library-GEMM form: [w_gu bf16 2 inter x hidden][w_d2 bf16 hidden x 2 inter]
// [g f32 T x 2 inter][a bf16 T x 2 inter]
struct SharedBlasWs {
  uint64_t w_gu, w_d2, g, a, total;
};

SharedBlasWs shared_blas_ws(uint32_t T, uint32_t hidden, uint32_t inter) {
  SharedBlasWs w;
  const uint64_t wb = 4ull * inter * hidden;
  w.w_gu = 0;
  w.w_d2 = a256(wb);
  w.g = w.w_d2 + a256(wb);
  w.a = w.g + a256(8ull * T * inter);
  w.total = w.a + a256(4ull * T * inter);
  return w;
}

// the batch's form: the library GEMMs unless AFFX_SHARED_BATCH=mfma asks for the fp8 MFMA kernels
bool shared_batch_mfma_only() {
  const char* v = getenv("AFFX_SHARED_BATCH");
  return v && strcmp(v, "mfma") == 0;
}

// The library-GEMM form of the batch: widen the three weight matrices to bf16 (gate rows then up
// rows in one [2 inter][hidden] matrix; down twice along K as [hidden][2 inter]); G = X W_gu^T
// (+ X_lo W_gu^T); the SwiGLU as two bf16 terms; y (+)= A W_d2^T, both terms summed by the GEMM.
// AFFX_DECLINED before y is touched when the library has no algorithm for a shape.
int shared_batch_blas(const affx_shared_expert* S, const void* x, const void* x_lo, uint32_t n_tok, float* y,
                      int accumulate, uint8_t* b, hipStream_t s) {
  const uint32_t H = S->hidden, I = S->inter;
  const SharedBlasWs lay = shared_blas_ws(n_tok, H, I);
  uint16_t* w_gu = (uint16_t*)(b + lay.w_gu);
  uint16_t* w_d2 = (uint16_t*)(b + lay.w_d2);
  float* g = (float*)(b + lay.g);
  uint16_t* a = (uint16_t*)(b + lay.a);
  WidenArgs W;
  const affx_dense_fp8* mats[3] = {&S->gate, &S->up, &S->down};
  for (int i = 0; i < 3; ++i) {
    W.w[i] = (const uint8_t*)mats[i]->data;
    W.s[i] = mats[i]->scales;
    W.rows[i] = i < 2 ? I : H;
    W.cols[i] = i < 2 ? H : I;
    W.ldo[i] = i < 2 ? H : 2u * I;
    W.copies[i] = i < 2 ? 1u : 2u;
    W.copy_off[i] = i < 2 ? 0u : I;
  }
  W.out[0] = w_gu;
  W.out[1] = w_gu + (uint64_t)I * H;
  W.out[2] = w_d2;
  W.wg_per = (uint32_t)((uint64_t)I * H / 16u / 256u);  // I * H is a multiple of 2^20
  hipLaunchKernelGGL(shexp_widen_kernel, dim3(3u * W.wg_per), dim3(256), 0, s, W);
  int rc = check_launch("shexp_widen_kernel");
  if (rc) return rc;
  if ((rc = blas_gemm_bf16_nt(2u * I, n_tok, H, w_gu, H, x, H, g, 2u * I, 0, s))) return rc;
  if (x_lo && (rc = blas_gemm_bf16_nt(2u * I, n_tok, H, w_gu, H, x_lo, H, g, 2u * I, 1, s))) return rc;
  const uint64_t quads = (uint64_t)n_tok * I / 4u;
  hipLaunchKernelGGL(shexp_swiglu_split_kernel, dim3((uint32_t)((quads + 255u) / 256u)), dim3(256), 0, s, g, a, I,
                     quads, S->swiglu_limit);
  if ((rc = check_launch("shexp_swiglu_split_kernel"))) return rc;
  return blas_gemm_bf16_nt(H, n_tok, 2u * I, w_d2, 2u * I, a, 2u * I, y, H, accumulate ? 1 : 0, s);
}

int shared_check(const affx_shared_expert* S, const char* what, uint32_t max_hidden) {
  if (!S) return set_error(AFFX_ERR_ARG, "%s: null shared expert", what);
  const affx_dense_fp8* m[3] = {&S->gate, &S->up, &S->down};
  for (int i = 0; i < 3; ++i) {
    if (!m[i]->data || !m[i]->scales) return set_error(AFFX_ERR_ARG, "%s: null weight or scale pointer", what);
    if ((reinterpret_cast<uintptr_t>(m[i]->data) & 15u) || (reinterpret_cast<uintptr_t>(m[i]->scales) & 3u))
      return set_error(AFFX_ERR_ARG, "%s: weights must be 16-byte and scales 4-byte aligned", what);
  }
  const uint32_t H = S->hidden, I = S->inter;
  if (S->gate.rows != I || S->gate.cols != H || S->up.rows != I || S->up.cols != H || S->down.rows != H ||
      S->down.cols != I)
    return set_error(AFFX_ERR_ARG, "%s: gate/up must be [inter x hidden] and down [hidden x inter]", what);
  if (H == 0 || I == 0 || H % kTileCols || I % kTileCols || H > max_hidden || I > 8192)
    return set_error(AFFX_DECLINED, "%s: hidden must be a multiple of 1024 up to %u and inter a multiple of 1024 "
                     "up to 8192 (got %u, %u)", what, max_hidden, H, I);
  if (!(S->swiglu_limit > 0.f) || S->swiglu_limit > 1e6f)
    return set_error(AFFX_DECLINED, "%s: needs a SwiGLU clamp limit in (0, 1e6]", what);
  return AFFX_OK;
}

template <int CG, bool VEC, int TOK>
void launch_gateup_form(uint32_t steps, dim3 g, hipStream_t s, const SharedArgs& A, const float* x, uint64_t xts,
                        uint64_t xds) {
  const dim3 b(kSxWaves * 64);
  switch (steps) {
    case 2: hipLaunchKernelGGL((shexp_gateup_kernel<CG, 2, VEC, TOK>), g, b, 0, s, A, x, xts, xds); break;
    case 4: hipLaunchKernelGGL((shexp_gateup_kernel<CG, 4, VEC, TOK>), g, b, 0, s, A, x, xts, xds); break;
    case 6: hipLaunchKernelGGL((shexp_gateup_kernel<CG, 6, VEC, TOK>), g, b, 0, s, A, x, xts, xds); break;
    default: hipLaunchKernelGGL((shexp_gateup_kernel<CG, 8, VEC, TOK>), g, b, 0, s, A, x, xts, xds); break;
  }
}

// (a kernel per activation form: the two load shapes under one runtime branch share a join)
template <int CG, int TOK>
void launch_gateup(uint32_t steps, dim3 g, hipStream_t s, const SharedArgs& A, const float* x, uint64_t xts,
                   uint64_t xds, int vec) {
  if (vec)
    launch_gateup_form<CG, true, TOK>(steps, g, s, A, x, xts, xds);
  else
    launch_gateup_form<CG, false, TOK>(steps, g, s, A, x, xts, xds);
}

template <int CG>
void launch_down(uint32_t steps, dim3 g, hipStream_t s, const SharedArgs& A) {
  switch (steps) {
    case 1: hipLaunchKernelGGL((shexp_down_kernel<CG, 1>), g, dim3(kSxWaves * 64), 0, s, A); break;
    case 2: hipLaunchKernelGGL((shexp_down_kernel<CG, 2>), g, dim3(kSxWaves * 64), 0, s, A); break;
    case 3: hipLaunchKernelGGL((shexp_down_kernel<CG, 3>), g, dim3(kSxWaves * 64), 0, s, A); break;
    case 4: hipLaunchKernelGGL((shexp_down_kernel<CG, 4>), g, dim3(kSxWaves * 64), 0, s, A); break;
    case 5: hipLaunchKernelGGL((shexp_down_kernel<CG, 5>), g, dim3(kSxWaves * 64), 0, s, A); break;
    case 6: hipLaunchKernelGGL((shexp_down_kernel<CG, 6>), g, dim3(kSxWaves * 64), 0, s, A); break;
    case 7: hipLaunchKernelGGL((shexp_down_kernel<CG, 7>), g, dim3(kSxWaves * 64), 0, s, A); break;
    default: hipLaunchKernelGGL((shexp_down_kernel<CG, 8>), g, dim3(kSxWaves * 64), 0, s, A); break;
  }
}

int hc_nh_ok(uint32_t n_hc, const char* what) {
  if (n_hc == 1 || n_hc == 2 || n_hc == 4 || n_hc == 8) return AFFX_OK;
  return set_error(AFFX_DECLINED, "%s: n_hc must be 1, 2, 4 or 8 (got %u)", what, n_hc);
}

}  // namespace

extern "C" {

size_t affx_shared_decode_workspace_size(uint32_t m_tokens, uint32_t hidden, uint32_t inter) {
  return (size_t)shared_decode_ws(m_tokens, hidden, inter).total;
}

size_t affx_shared_batch_workspace_size(uint32_t n_tok, uint32_t hidden, uint32_t inter) {
  const uint64_t own = shared_batch_ws(n_tok, hidden, inter).total, lib = shared_blas_ws(n_tok, hidden, inter).total;
  return (size_t)(own > lib ? own : lib);
}

int affx_shared_expert_decode(const affx_shared_expert* S, const float* x, uint64_t x_ts, uint64_t x_ds,
                              uint32_t m_tokens, float* y, uint64_t y_ts, uint64_t y_ds, int accumulate, void* ws,
                              size_t ws_bytes, void* stream) {
  int rc = shared_check(S, "shared_expert_decode", 4 * kTileCols);
  if (rc) return rc;
  if (!x || !y || !ws) return set_error(AFFX_ERR_ARG, "shared_expert_decode: null pointer");
  if (m_tokens == 0 || m_tokens > (uint32_t)kMaxTok)
    return set_error(AFFX_DECLINED, "shared_expert_decode: m_tokens must be 1..%d (got %u)", kMaxTok, m_tokens);
  const SharedWs lay = shared_decode_ws(m_tokens, S->hidden, S->inter);
  if (ws_bytes < lay.total)
    return set_error(AFFX_ERR_ARG, "shared_expert_decode: workspace %zu < %llu bytes", ws_bytes,
                     (unsigned long long)lay.total);
  uint8_t* b = (uint8_t*)ws;
  hipStream_t s = (hipStream_t)stream;
  SharedArgs A;
  A.w[0] = (const uint8_t*)S->gate.data; A.s[0] = S->gate.scales;
  A.w[1] = (const uint8_t*)S->up.data;   A.s[1] = S->up.scales;
  A.w[2] = (const uint8_t*)S->down.data; A.s[2] = S->down.scales;
  A.hidden = S->hidden;
  A.inter = S->inter;
  A.m_tokens = m_tokens;
  A.aq = b + lay.aq;
  A.limit = S->swiglu_limit;
  A.sigma_a = 7 - ilogbf(S->swiglu_limit * S->swiglu_limit);
  A.y = y;
  A.y_ts = y_ts;
  A.y_ds = y_ds;
  A.accumulate = accumulate;
  const uint32_t gsteps = S->hidden / 512u, dsteps = S->inter / 1024u;
  // token-major rows with 16-byte alignment take 16-byte loads, any other strides element loads
  const int vec = x_ds == 1 && (x_ts % 4) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  if (m_tokens <= 5) {
    if (m_tokens == 1)
      launch_gateup<1, 1>(gsteps, dim3(S->inter / 8u), s, A, x, x_ts, x_ds, vec);
    else
      launch_gateup<1, 5>(gsteps, dim3(S->inter / 8u), s, A, x, x_ts, x_ds, vec);
    if ((rc = check_launch("shexp_gateup_kernel"))) return rc;
    launch_down<1>(dsteps, dim3(S->hidden / 16u), s, A);
  } else {
    launch_gateup<2, kMaxTok>(gsteps, dim3(S->inter / 8u), s, A, x, x_ts, x_ds, vec);
    if ((rc = check_launch("shexp_gateup_kernel"))) return rc;
    launch_down<2>(dsteps, dim3(S->hidden / 16u), s, A);
  }
  return check_launch("shexp_down_kernel");
}

int affx_shared_expert_batch(const affx_shared_expert* S, const void* x, const void* x_lo, uint32_t n_tok, float* y,
                             int accumulate, void* ws, size_t ws_bytes, void* stream) {
  int rc = shared_check(S, "shared_expert_batch", 8192);
  if (rc) return rc;
  if (!x || !y || !ws) return set_error(AFFX_ERR_ARG, "shared_expert_batch: null pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(x_lo) | reinterpret_cast<uintptr_t>(y) |
       reinterpret_cast<uintptr_t>(ws)) & 15u)
    return set_error(AFFX_ERR_ARG, "shared_expert_batch: x, x_lo, y and the workspace must be 16-byte aligned");
  if (n_tok == 0) return AFFX_OK;
  const SharedWs lay = shared_batch_ws(n_tok, S->hidden, S->inter);
  const uint64_t need = affx_shared_batch_workspace_size(n_tok, S->hidden, S->inter);
  if (lay.total > (1ull << 32) || need > (1ull << 33))
    return set_error(AFFX_DECLINED, "shared_expert_batch: batch too large (split it)");
  if (ws_bytes < need)
    return set_error(AFFX_ERR_ARG, "shared_expert_batch: workspace %zu < %llu bytes", ws_bytes,
                     (unsigned long long)need);
  uint8_t* b = (uint8_t*)ws;
  hipStream_t s = (hipStream_t)stream;
  if (!shared_batch_mfma_only()) {
    rc = shared_batch_blas(S, x, x_lo, n_tok, y, accumulate, b, s);
    if (rc != AFFX_DECLINED) return rc;
  }
  // the fp8 MFMA kernels (a shape the library declines, or asked for by name)
  const uint32_t tx = x_lo ? 3 : 2;
  const uint32_t zmax = S->hidden > S->inter ? S->hidden : S->inter;
  hipLaunchKernelGGL(shexp_prep_rows_kernel, dim3(n_tok), dim3(256), 0, s, (const uint16_t*)x, (const uint16_t*)x_lo,
                     S->hidden, tx, (int32_t*)(b + lay.sigma), b + lay.xq, (uint32_t*)(b + lay.zeros), zmax / 4);
  if ((rc = check_launch("shexp_prep_rows_kernel"))) return rc;
  SharedGemmArgs A;
  A.n_tok = n_tok;
  A.ws = b;
  A.zero_off = lay.zeros;
  A.sigma = (const int32_t*)(b + lay.sigma);
  A.sigma_a = 7 - ilogbf(S->swiglu_limit * S->swiglu_limit);
  A.inter = S->inter;
  A.hidden = S->hidden;
  A.aq = b + lay.aq;
  A.y = y;
  A.accumulate = accumulate;
  A.limit = S->swiglu_limit;
  // gate/up: 128 rows of inter per item
  A.w0 = (const uint8_t*)S->gate.data; A.s0 = S->gate.scales;
  A.w1 = (const uint8_t*)S->up.data;   A.s1 = S->up.scales;
  A.K = S->hidden;
  A.b_off = lay.xq;
  A.n_rb = S->inter / 128u;
  A.n_tiles = (n_tok + (uint32_t)kBCT * (16u / tx) - 1u) / ((uint32_t)kBCT * (16u / tx));
  dim3 g(8u * ((A.n_rb + 7u) / 8u) * A.n_tiles);
  if (tx == 2)
    hipLaunchKernelGGL((shexp_gemm_kernel<0, 2>), g, dim3(kBT), 0, s, A);
  else
    hipLaunchKernelGGL((shexp_gemm_kernel<0, 3>), g, dim3(kBT), 0, s, A);
  if ((rc = check_launch("shexp_gemm_kernel (gate/up)"))) return rc;
  // down: 256 rows of hidden per item, the SwiGLU output's three terms
  A.w0 = (const uint8_t*)S->down.data; A.s0 = S->down.scales;
  A.w1 = nullptr; A.s1 = nullptr;
  A.K = S->inter;
  A.b_off = lay.aq;
  A.n_rb = S->hidden / 256u;
  A.n_tiles = (n_tok + (uint32_t)kBCT * 5u - 1u) / ((uint32_t)kBCT * 5u);
  g = dim3(8u * ((A.n_rb + 7u) / 8u) * A.n_tiles);
  hipLaunchKernelGGL((shexp_gemm_kernel<1, 3>), g, dim3(kBT), 0, s, A);
  return check_launch("shexp_gemm_kernel (down)");
}

int affx_dense_fp8_to_device_layout(const void* src, void* dst, uint64_t rows, uint64_t cols, void* stream) {
  if (!src || !dst) return set_error(AFFX_ERR_ARG, "dense_fp8_to_device_layout: null pointer");
  if (rows == 0 || cols == 0 || rows % 16 || cols % 128 || rows * cols > 0xFFFFFFFFull ||
      ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u))
    return set_error(AFFX_ERR_ARG, "dense_fp8_to_device_layout: rows must be a multiple of 16, cols of 128, "
                     "rows*cols < 4 GiB, both buffers 16-byte aligned");
  if (src == dst) return set_error(AFFX_ERR_ARG, "dense_fp8_to_device_layout: src and dst must differ");
  const uint64_t chunks = rows * cols / 16u;
  hipLaunchKernelGGL(dense_fp8_permute_kernel, dim3((uint32_t)((chunks + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)src, (uint8_t*)dst, (uint32_t)rows, (uint32_t)cols);
  return check_launch("dense_fp8_permute_kernel");
}

int affx_hc_post(float* out_hc, float* block, const float* hc, const float* post, const float* comb,
                 uint32_t n_embd, uint32_t n_hc, int zero_block, void* stream) {
  if (!out_hc || !block || !hc || !post || !comb) return set_error(AFFX_ERR_ARG, "hc_post: null pointer");
  int rc = hc_nh_ok(n_hc, "hc_post");
  if (rc) return rc;
  if (n_embd == 0) return AFFX_OK;
  const dim3 g((n_embd + 255) / 256), t(256);
  hipStream_t s = (hipStream_t)stream;
  switch (n_hc) {
    case 1: hipLaunchKernelGGL(hc_expand_kernel<1>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, zero_block); break;
    case 2: hipLaunchKernelGGL(hc_expand_kernel<2>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, zero_block); break;
    case 4: hipLaunchKernelGGL(hc_expand_kernel<4>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, zero_block); break;
    default: hipLaunchKernelGGL(hc_expand_kernel<8>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, zero_block); break;
  }
  return check_launch("hc_expand_kernel");
}

int affx_hc_add(float* hc, float* block, uint32_t n_embd, int zero_block, void* stream) {
  if (!hc || !block) return set_error(AFFX_ERR_ARG, "hc_add: null pointer");
  if (n_embd == 0) return AFFX_OK;
  hipLaunchKernelGGL(hc_add_kernel, dim3((n_embd + 255) / 256), dim3(256), 0, (hipStream_t)stream, hc, block,
                     (uint64_t)n_embd, zero_block);
  return check_launch("hc_add_kernel");
}

int affx_hc_post_batch(uint16_t* out_hc, float* block, const uint16_t* hc, const float* post, const float* comb,
                       uint32_t n_embd, uint32_t n_hc, uint32_t nb, int zero_block, void* stream) {
  if (!out_hc || !block || !hc || !post || !comb) return set_error(AFFX_ERR_ARG, "hc_post_batch: null pointer");
  int rc = hc_nh_ok(n_hc, "hc_post_batch");
  if (rc) return rc;
  const uint64_t total = (uint64_t)n_embd * nb;
  if (total == 0) return AFFX_OK;
  if ((total + 255) / 256 > 0x7FFFFFFFull) return set_error(AFFX_DECLINED, "hc_post_batch: arena too large");
  const dim3 g((uint32_t)((total + 255) / 256)), t(256);
  hipStream_t s = (hipStream_t)stream;
  switch (n_hc) {
    case 1: hipLaunchKernelGGL(hc_expand_batch_kernel<1>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, nb, zero_block); break;
    case 2: hipLaunchKernelGGL(hc_expand_batch_kernel<2>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, nb, zero_block); break;
    case 4: hipLaunchKernelGGL(hc_expand_batch_kernel<4>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, nb, zero_block); break;
    default: hipLaunchKernelGGL(hc_expand_batch_kernel<8>, g, t, 0, s, out_hc, block, hc, post, comb, n_embd, nb, zero_block); break;
  }
  return check_launch("hc_expand_batch_kernel");
}

int affx_hc_add_batch(uint16_t* hc, float* block, uint64_t n, int zero_block, void* stream) {
  if (!hc || !block) return set_error(AFFX_ERR_ARG, "hc_add_batch: null pointer");
  if (n == 0) return AFFX_OK;
  if ((n + 255) / 256 > 0x7FFFFFFFull) return set_error(AFFX_DECLINED, "hc_add_batch: arena too large");
  hipLaunchKernelGGL(hc_add_batch_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, hc,
                     block, n, zero_block);
  return check_launch("hc_add_batch_kernel");
}

}  // extern "C"
