// Device pieces shared by the decode GEMV and the grouped prefill GEMM: loading a wave tile's
// packed units, the LDS codebook, and decoding an MFMA A fragment from packed codes.
#pragma once

#include "affx_common.h"

namespace affx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// a unit's 12-byte field run (4-byte aligned): one global_load_dwordx3
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));

// ------------------------------------------------------------------------------------------------
// shared pieces of the GEMV and GEMM kernels
// ------------------------------------------------------------------------------------------------

// A unit's packed data: 20 code dwords + 3 field dwords.
struct Unit {
  uint32_t c[20];
  uint32_t f[3];
};

__device__ __forceinline__ void load_unit(Unit& u, const uint8_t* codes, const uint8_t* fields,
                                          uint64_t tile, uint32_t lane) {
  const uint8_t* cp = codes + tile * kTileCodeBytes + lane * 16;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cp + j * 1024));
    u.c[4 * j] = v[0]; u.c[4 * j + 1] = v[1]; u.c[4 * j + 2] = v[2]; u.c[4 * j + 3] = v[3];
  }
  const uint32_t* fp = reinterpret_cast<const uint32_t*>(fields + tile * kTileFieldBytes + lane * 12);
  u.f[0] = __builtin_nontemporal_load(fp);
  u.f[1] = __builtin_nontemporal_load(fp + 1);
  u.f[2] = __builtin_nontemporal_load(fp + 2);
}

// Makes the unit's registers opaque at this point of the program. Called at the top of every
// MFMA step, it stops the compiler from hoisting all eight steps' code extraction and address
// arithmetic (pure ALU, free to move) in front of the first step, which would keep ~100 extra
// VGPRs live and halve occupancy. No instructions are emitted.
#ifndef AFFX_PIN
#define AFFX_PIN(x) asm volatile("" : "+v"(x))
#endif
// Cross-lane moves within a row of 16 lanes, as one DPP op (not an LDS permute): lane l gets the
// value of lane l + N (row_shl) or l - N (row_shr) of its row; a lane whose source is outside
// the row keeps its own value.
template <int N>
__device__ __forceinline__ float row_shl(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x100 + N, 0xF, 0xF, false));
}
template <int N>
__device__ __forceinline__ float row_shr(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x110 + N, 0xF, 0xF, false));
}
// Buffer resource over `bytes` bytes at p (raw buffer, no swizzle; reads past the end return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// Cache policy of a buffer access that must see, or be seen by, other workgroups on any XCD
// without a fence: the device-scope coherence bit (sc1 on gfx950), as the compiler emits it for
// an agent-scope atomic load or store.
constexpr int kDevCoherent = 16;
// LDS pointer operand of a direct global->LDS load.
#ifndef AFFX_LDS_PTR
#define AFFX_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))
#endif
__device__ __forceinline__ void pin(Unit& u) {
#pragma unroll
  for (int i = 0; i < 20; ++i) AFFX_PIN(u.c[i]);
#pragma unroll
  for (int i = 0; i < 3; ++i) AFFX_PIN(u.f[i]);
}

// The A fragment of MFMA step m: codes 8m..8m+7 of the unit (blocks 2m, 2m+1), each looked up
// in the LDS table of its block's (variant, rotation) and xor/add-transformed.
template <int MSTEP>
__device__ __forceinline__ v8i decode_a(const Unit& u, const uint32_t* tbl) {
  v8i a;
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    const int b = 2 * MSTEP + bb;
    const uint32_t fb = stream_bits<3>(u.f, 6 * b, 6);
    const uint32_t base = (fb >> 4) << 10;
    const uint32_t x = block_xor(fb), ad = block_add(fb);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t code = stream_bits<20>(u.c, 10 * (4 * b + i), 10);
      a[bb * 4 + i] = (int)((tbl[base + code] ^ x) + ad);
    }
  }
  return a;
}

// decode_a in two halves, so that the LDS lookups of step m+1 can be in flight while step m is
// finished and multiplied: lookup_a issues the eight table reads, finish_a applies each block's
// sign and exponent add.
template <int MSTEP>
__device__ __forceinline__ void lookup_a(const Unit& u, const uint32_t* tbl, uint32_t (&raw)[8]) {
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    const int b = 2 * MSTEP + bb;
    const uint32_t base = (stream_bits<3>(u.f, 6 * b, 6) >> 4) << 10;
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[bb * 4 + i] = tbl[base + stream_bits<20>(u.c, 10 * (4 * b + i), 10)];
  }
}

template <int MSTEP>
__device__ __forceinline__ v8i finish_a(const Unit& u, const uint32_t (&raw)[8]) {
  v8i a;
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    const uint32_t fb = stream_bits<3>(u.f, 6 * (2 * MSTEP + bb), 6);
    const uint32_t x = block_xor(fb), ad = block_add(fb);
#pragma unroll
    for (int i = 0; i < 4; ++i) a[bb * 4 + i] = (int)((raw[bb * 4 + i] ^ x) + ad);
  }
  return a;
}

__device__ __forceinline__ void lookup_step(const Unit& u, const uint32_t* tbl, int m, uint32_t (&raw)[8]) {
  switch (m) {
    case 0: lookup_a<0>(u, tbl, raw); break;
    case 1: lookup_a<1>(u, tbl, raw); break;
    case 2: lookup_a<2>(u, tbl, raw); break;
    case 3: lookup_a<3>(u, tbl, raw); break;
    case 4: lookup_a<4>(u, tbl, raw); break;
    case 5: lookup_a<5>(u, tbl, raw); break;
    case 6: lookup_a<6>(u, tbl, raw); break;
    default: lookup_a<7>(u, tbl, raw); break;
  }
}

__device__ __forceinline__ v8i finish_step(const Unit& u, int m, const uint32_t (&raw)[8]) {
  switch (m) {
    case 0: return finish_a<0>(u, raw);
    case 1: return finish_a<1>(u, raw);
    case 2: return finish_a<2>(u, raw);
    case 3: return finish_a<3>(u, raw);
    case 4: return finish_a<4>(u, raw);
    case 5: return finish_a<5>(u, raw);
    case 6: return finish_a<6>(u, raw);
    default: return finish_a<7>(u, raw);
  }
}

// decode_a with a step index that is a compile-time constant after unrolling.
__device__ __forceinline__ v8i decode_step(const Unit& u, const uint32_t* tbl, int m) {
  switch (m) {
    case 0: return decode_a<0>(u, tbl);
    case 1: return decode_a<1>(u, tbl);
    case 2: return decode_a<2>(u, tbl);
    case 3: return decode_a<3>(u, tbl);
    case 4: return decode_a<4>(u, tbl);
    case 5: return decode_a<5>(u, tbl);
    case 6: return decode_a<6>(u, tbl);
    default: return decode_a<7>(u, tbl);
  }
}

// Three E4M3 terms of v (|v| < 448): v ~= e(b0) + e(b1)/16 + e(b2)/256, residual <= 2^-12 |v|
// for v in E4M3's normal range.
__device__ __forceinline__ void split3(float v, uint32_t& b0, uint32_t& b1, uint32_t& b2) {
  b0 = f32_to_e4m3(v);
  const float r1 = (v - e4m3_to_f32(b0)) * 16.0f;
  b1 = f32_to_e4m3(r1);
  const float r2 = (r1 - e4m3_to_f32(b1)) * 16.0f;
  b2 = f32_to_e4m3(r2);
}

// One (token t, 1024-column super-segment S) of the decode input x (f32, element (t, h) at
// x[t * xts + h * xds]): its exponent sigma (returned: the segment's largest magnitude times
// 2^sigma lies in [128, 256), below E4M3's 448 with one binade of headroom) and three E4M3 terms
// of every element times 2^sigma, natural column order, term j at xq + (3 t + j) * hidden + h
// (nothing written when xq is null). All 256 threads of the workgroup call it (red: 4 floats of
// LDS). In two parts, so that a caller can issue the loads before others and split later.
__device__ __forceinline__ void segment_load(const float* __restrict__ x, uint64_t xts, uint64_t xds, uint32_t t,
                                             uint32_t S, float (&v)[4]) {
  const uint32_t h0 = S * kTileCols + 4 * threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = x[t * xts + (h0 + i) * xds];
}
__device__ __forceinline__ int segment_split(const float (&v)[4], uint32_t t, uint32_t S, uint32_t hidden,
                                             uint8_t* xq, float* red) {
  const uint32_t tid = threadIdx.x;
  const uint32_t h0 = S * kTileCols + 4 * tid;
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(v[i]));
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int sigma = amax > 0.f ? 7 - ilogbf(amax) : 0;
  if (xq) {
    uint32_t q0 = 0, q1 = 0, q2 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t b0, b1, b2;
      split3(ldexpf(v[i], sigma), b0, b1, b2);
      q0 |= b0 << (8 * i);
      q1 |= b1 << (8 * i);
      q2 |= b2 << (8 * i);
    }
    uint32_t* dst = reinterpret_cast<uint32_t*>(xq + (uint64_t)t * kTerms * hidden + h0);
    dst[0] = q0;
    dst[hidden / 4] = q1;
    dst[2 * (hidden / 4)] = q2;
  }
  return sigma;
}
__device__ __forceinline__ int segment_terms(const float* __restrict__ x, uint64_t xts, uint64_t xds, uint32_t t,
                                             uint32_t S, uint32_t hidden, uint8_t* xq, float* red) {
  float v[4];
  segment_load(x, xts, xds, t, S, v);
  return segment_split(v, t, S, hidden, xq, red);
}

// B operand of one unit: per lane, 256 consecutive activation bytes of one (token, term) column
// (MFMA step m reads bytes 32m..32m+31). Lanes whose column is unused (column 15, tokens beyond
// M or not routed to this expert) read nothing and feed zeros.
template <int CG>
struct BSrc {
  const u32x4* p[CG];
  bool used;  // (column group 0) this lane's column is a used (token, term) column
};

template <int CG>
__device__ __forceinline__ BSrc<CG> b_source(const uint8_t* src_base, uint64_t term_stride,
                                             uint64_t col0, uint32_t lane, uint32_t M,
                                             uint32_t mask, const uint8_t* zeros) {
  BSrc<CG> s;
  const uint32_t c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const uint32_t t = cg * 5 + c / 3, tau = c % 3;
    const bool valid = c < 15 && t < M && ((mask >> t) & 1u);
    s.p[cg] = valid ? reinterpret_cast<const u32x4*>(src_base + (uint64_t)(t * kTerms + tau) * term_stride +
                                                     col0 + g * kSegCols)
                    : reinterpret_cast<const u32x4*>(zeros);
    if (cg == 0) s.used = valid;
  }
  return s;
}

__device__ __forceinline__ v8i b_step(const u32x4* p, int m) {
  const u32x4 lo = p[2 * m], hi = p[2 * m + 1];
  v8i v;
  v[0] = (int)lo[0]; v[1] = (int)lo[1]; v[2] = (int)lo[2]; v[3] = (int)lo[3];
  v[4] = (int)hi[0]; v[5] = (int)hi[1]; v[6] = (int)hi[2]; v[7] = (int)hi[3];
  return v;
}

__device__ __forceinline__ v4f mfma(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// LDS codebook: table t = rot + 2*variant (= field >> 4), entry c = codebook dword, rotated by
// 16 bits for rot = 1 (quad (a,b,c,d) read as (c,d,a,b): src/quant/blockquant.cpp:826-828).
__device__ __forceinline__ void build_table(uint32_t* tbl, const uint32_t* __restrict__ cb) {
  for (uint32_t i = threadIdx.x; i < kVariants * kLut; i += blockDim.x) {
    const uint32_t d = cb[i], v = i >> 10, c = i & 1023u;
    tbl[(2 * v) * kLut + c] = d;
    tbl[(2 * v + 1) * kLut + c] = __builtin_amdgcn_alignbit(d, d, 16);
  }
}

}  // namespace affx
