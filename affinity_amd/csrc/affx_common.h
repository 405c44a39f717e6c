// Shared definitions of libaffx.so (gfx950, wave64). Device layout, fp8 helpers, status plumbing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/affx.h"

namespace affx {

// ---- format (AFF_Q2P875_Q4): block 16, 10-bit quad codes, 6-bit fields, bf16 row scale -------
// src/quant/blockquant.cpp:22-30, src/format/aff_format.h:117-121
constexpr int kBlock = 16;
constexpr int kLut = 1024;
constexpr int kVariants = 2;

// ---- device layout ---------------------------------------------------------------------------
// A "unit" is one row's 256-column segment: 80 bytes of codes (64 codes) + 12 bytes of fields
// (16 fields), a contiguous byte run of each row-major stream. A wave tile is 16 rows x 1024
// columns = 64 units, one per lane: lane = (row % 16) + 16 * (segment % 4). Tiles are stored
// row-tile major, column-tile minor: tile (rt, st) at index rt * (cols / 1024) + st. Inside a
// tile the code plane holds five 1 KiB chunks [chunk j][lane][16 B] (chunk j = unit bytes
// 16j..16j+15) and the field plane one 768 B run [lane][12 B].
constexpr int kTileRows = 16;
constexpr int kTileCols = 1024;
constexpr int kSegCols = 256;
constexpr int kUnitCodeBytes = 80;
constexpr int kUnitFieldBytes = 12;
constexpr int kTileCodeBytes = 64 * kUnitCodeBytes;    // 5120
constexpr int kTileFieldBytes = 64 * kUnitFieldBytes;  // 768

// Index of each plane in the off9/size9 arrays of affx_expert_layout: matrix-major
// (gate, up, down), plane-minor (codes, fields, row scales).
enum Plane : int {
  kGateCodes = 0, kGateFields = 1, kGateRs = 2,
  kUpCodes = 3, kUpFields = 4, kUpRs = 5,
  kDownCodes = 6, kDownFields = 7, kDownRs = 8
};

__host__ __device__ inline uint64_t a256(uint64_t v) { return (v + 255) / 256 * 256; }
__host__ __device__ inline uint64_t code_row_bytes(uint64_t cols) { return cols * 10 / 32; }
__host__ __device__ inline uint64_t field_row_bytes(uint64_t cols) { return cols * 6 / 128; }

// ---- activations as exact fp8 sums -------------------------------------------------------------
// An activation v is fed to the fp8 MFMA as kTerms E4M3 values: v * 2^sigma ~= t0 + t1/16 +
// t2/256, each term in its own B column. Residual after three terms <= 2^-12 relative.
constexpr int kTerms = 3;
constexpr int kMaxTok = AFFX_MAX_DECODE_TOKENS;
constexpr int kMaxSlots = AFFX_MAX_DECODE_TOKENS * AFFX_MAX_TOPK;  // distinct experts of a batch

// Plan the decode prep kernel writes: the distinct experts of the batch (ascending id), which
// tokens each one serves and with what weight, and the exponent of every activation segment.
constexpr int kMaxSeg = 4;  // 1024-column super-segments of the decode input (hidden <= 4096)

struct DecodePlan {
  uint32_t n_slots;
  uint32_t m_tokens;
  int32_t x_sigma[kMaxTok][kMaxSeg];  // exponent of each (token, super-segment) activation split
  uint32_t expert[kMaxSlots];
  uint32_t tok_mask[kMaxSlots];
  float w[kMaxSlots][kMaxTok];  // last: a plan of n slots ends at w[n] (the pointer-table form's scratch)
};
static_assert(offsetof(DecodePlan, w) + sizeof(float) * kMaxSlots * kMaxTok == sizeof(DecodePlan),
              "the weight table ends the plan");

// Phase markers of the persistent decode kernel: expand to nothing (a profiling build can define
// them to record timestamps).
#ifndef AFFX_TRACE
#define AFFX_TRACE(k) ((void)0)
#endif
#ifndef AFFX_TRACEW
#define AFFX_TRACEW(k) ((void)0)
#endif
#ifndef AFFX_TRACE_INIT
#define AFFX_TRACE_INIT ((void)0)
#endif

// waitcnt immediate for "at most n vector memory operations outstanding" (gfx9 encoding; the
// other counters left at their maxima)
#define AFFX_VMCNT(n) ((((n) & 15) | (((n) >> 4) << 14)) | (0x7 << 4) | (0xF << 8))

// Dynamic LDS of a kernel (one byte array; the kernel carves it up).
#ifndef AFFX_DYN_LDS
#define AFFX_DYN_LDS(name) extern __shared__ __align__(16) uint8_t name[]
#endif

// Decode workspace: [sync][plan][zeros][xq][aq] (affx_decode.hip). The sync run holds the fused
// decode's cross-workgroup state:
//  * a 256-byte header: dword 0 gate/up items published (rounds kernels), dword 2 error bits,
//    dword 8 the launch epoch of the one-pass (batch-1) kernel;
//  * one release flag per waiting workgroup, 128 bytes apart so that no two workgroups poll the
//    same line (rounds kernels);
//  * the one-pass kernel's publish flags: kPubReplicas copies of one dword per workgroup, each
//    copy a kPubStride run, holding the epoch in which that workgroup's SwiGLU output was last
//    complete.
// Zero before first use. Every launch leaves the counter and the release flags zero; the epoch
// and the publish flags only ever advance (zero is their state after a reset as well).
constexpr uint32_t kSyncHeader = 256;
constexpr uint32_t kSyncFlagStride = 128;
constexpr uint32_t kSyncFlags = 256;  // down-phase workgroups: output row tiles, hidden / 16 <= 256
constexpr uint32_t kSyncRunBytes = kSyncHeader + kSyncFlags * kSyncFlagStride;
constexpr uint32_t kPubReplicas = 8;  // one per XCD: a waiter polls copy g % 8
constexpr uint32_t kPubStride = 1024; // bytes per copy: 256 workgroups
constexpr uint32_t kPubOff = kSyncRunBytes;
constexpr uint32_t kSyncBytes = kPubOff + kPubReplicas * kPubStride;
constexpr uint32_t kSyncErrWord = 2;  // dword of the error bits (bit 0: a waiter gave up)
constexpr uint32_t kEpochWord = 8;    // dword of the one-pass kernel's launch epoch
// Zeroes the sync run of a decode workspace (stream-ordered; after a wait gave up, the late
// publisher may have raised flags that a later launch would take for its own).
int decode_sync_reset(void* ws, hipStream_t s);
struct DecodeWs {
  uint64_t sync, plan, zeros, xq, aq, total;
};
DecodeWs decode_ws(uint32_t M, uint32_t K, uint32_t hidden, uint32_t inter);
int decode_check(const affx_layer* L, uint32_t M, uint32_t K, const void* ws, size_t ws_bytes,
                 DecodeWs* lay);

// Set-up of the allocation-free decode's scratch array on device `dev` (current), from affx_init.
int noalloc_init_device(int dev);

// ---- plain bf16 GEMM (hipBLASLt; affx_blas.cpp) -------------------------------------------------
// D[n][m] = sum_k A[m][k] B[n][k] (+ D[n][m] when beta_one), f32 accumulation and output: A [M][K]
// and B [N][K] bf16 row-major with row strides lda, ldb (elements), D [N][M] f32 with row stride
// ldd. AFFX_DECLINED, with nothing enqueued, when the library has no algorithm for the shape. The
// first call for a shape asks the library's heuristic on the host (not under graph capture).
int blas_gemm_bf16_nt(uint32_t M, uint32_t N, uint32_t K, const void* A, uint32_t lda, const void* B, uint32_t ldb,
                      float* D, uint32_t ldd, int beta_one, hipStream_t stream);

// ---- status ------------------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
int check_launch(const char* what);

// ---- device helpers ----------------------------------------------------------------------------

// Lanes of this wave whose BITS-bit key equals this lane's, among `valid` ones (one ballot per key
// bit: a fixed cost, whatever the number of distinct keys).
template <int BITS>
__device__ __forceinline__ uint64_t same_key_lanes(uint32_t k, bool valid) {
  uint64_t m = __ballot(valid);
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    const uint32_t bit = (k >> b) & 1u;
    const uint64_t bal = __ballot(bit);
    m &= bit ? bal : ~bal;
  }
  return m;
}

// Exact E4M3 (OCP fn) -> f32 for a non-NaN byte.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;
  return __uint_as_float(__float_as_uint(v) | ((b & 0x80u) << 24));
}

// f32 -> E4M3 (OCP fn), round to nearest even, saturating at +-448 (never NaN).
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
  const uint32_t s = (__float_as_uint(v) >> 24) & 0x80u;
  const float a = fabsf(v);
  if (!(a < 464.0f)) return s | 0x7Eu;
  if (a < 0.015625f) return s | (uint32_t)rintf(a * 512.0f);  // 8 -> 0x08, the least normal
  const uint32_t au = __float_as_uint(a);
  int e = (int)(au >> 23) - 127;
  uint32_t m3 = (au >> 20) & 7u;
  const uint32_t rem = au & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) {
    if (++m3 == 8u) { m3 = 0; ++e; }
  }
  return s | ((uint32_t)(e + 7) << 3) | m3;
}

// The packed-dword block transform of the reference decode (src/gpu/expert_kernel.hip:594-617):
// sign = XOR 0x80 per byte, block scale 2^s = +s on every byte's exponent (stored exponent 1..7
// plus s <= 7 stays <= 14: no carry, never NaN). Rotation is applied by table choice.
__device__ __forceinline__ uint32_t block_xor(uint32_t f) { return (f & 8u) ? 0x80808080u : 0u; }
__device__ __forceinline__ uint32_t block_add(uint32_t f) {
  return __builtin_amdgcn_perm(0u, (f & 7u) << 3, 0u);  // (s<<3) replicated into all 4 bytes
}

// Bits [pos, pos+n) of a little-endian stream held in registers (pos, n compile-time after
// unrolling).
template <int N>
__device__ __forceinline__ uint32_t stream_bits(const uint32_t* d, int pos, int n) {
  const int i = pos >> 5, sh = pos & 31;
  uint32_t v = d[i] >> sh;
  if (sh + n > 32 && i + 1 < N) v = __builtin_amdgcn_alignbit(d[i + 1], d[i], sh);
  return v & ((1u << n) - 1u);
}

}  // namespace affx
