// The replicated LDS codebook and the A-fragment decode shared by the one-launch decode and the
// grouped prefill GEMM: a lane's unit (one row's 256-column segment) is looked up code by code in
// one of KC interleaved copies of the codebook and turned into an E4M3 MFMA A fragment.
#pragma once

#include "affx_tile.h"

namespace affx {

// ---- replicated codebook -------------------------------------------------------------------------
// KC interleaved copies of the 2 x 1024 codebook dwords: entry (variant v, code c) of copy j at
// dword ((v << 10 | c) * KC + j). A lane reads copy (lane >> 1) % KC, so the 64 gathers of one
// instruction spread over the banks by lane instead of colliding at random. With ROT the table
// also holds every dword pre-rotated (the block rotation of blockquant.cpp:826-828): table
// t = 2v + rot, entry (t, c) of copy j at dword ((t << 10 | c) * KC + j), so a lookup needs no
// rotate (twice the LDS).
template <int KC, bool ROT = false>
struct Lut {
  static constexpr int kLog = KC == 16 ? 4 : KC == 8 ? 3 : KC == 4 ? 2 : 1;
  static constexpr int kCodeSh = kLog + 2;       // byte-address bit of code bit 0
  static constexpr int kVarSh = kCodeSh + 10;    // byte-address bit of the table index
  static constexpr int kDwords = KC * (ROT ? 4096 : 2048);
};

// (thread i0 of NT: entries i0 + NT * i, i < N; cbv[i] = codebook dword of that entry)
template <int KC, int NT, int N, bool ROT = false>
__device__ __forceinline__ void build_lut(uint32_t* tbl, const uint32_t (&cbv)[N], uint32_t i0) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t e = i0 + (uint32_t)i * NT;
    if (e >= 2048u) break;
    const uint32_t d = cbv[i];
    auto put = [&](uint32_t idx, uint32_t val) {
      if constexpr (KC >= 4) {
        const u32x4 v = {val, val, val, val};
        u32x4* dst = reinterpret_cast<u32x4*>(tbl + idx * KC);
#pragma unroll
        for (int q = 0; q < KC / 4; ++q) dst[q] = v;
      } else {
#pragma unroll
        for (int q = 0; q < KC; ++q) tbl[idx * KC + q] = val;
      }
    };
    if constexpr (ROT) {
      const uint32_t v = e >> 10, c = e & 1023u;
      put((2u * v) << 10 | c, d);
      put((2u * v + 1u) << 10 | c, __builtin_amdgcn_alignbit(d, d, 16));
    } else {
      put(e, d);
    }
  }
}

// LDS byte address of code I (0..63) of the unit: the code's ten bits are brought to bit kCodeSh
// of an alignbit window and inserted into vb (the block's variant and the lane's copy; bits
// outside the code field come from vb).
template <int KC, int I>
__device__ __forceinline__ uint32_t code_addr(const uint32_t (&c)[20], uint32_t vb) {
  constexpr int S = Lut<KC>::kCodeSh;  // (the same with or without rotated tables)
  constexpr int q = 10 * I - S;
  uint32_t x;
  if constexpr (q < 0) {
    x = __builtin_amdgcn_alignbit(c[0], c[0], q + 32);
  } else {
    constexpr int lo = q >> 5, sh = q & 31;
    constexpr int hi = (sh + S + 10 > 32 && lo + 1 < 20) ? lo + 1 : lo;
    x = sh == 0 ? c[lo] : __builtin_amdgcn_alignbit(c[hi], c[lo], sh);
  }
  return (x & (0x3FFu << S)) | vb;
}

// Sign mask and exponent add of a block by the low four bits of its field (bits 0-2 exponent add
// s, bit 3 sign): entry f = {sign ? 0x80808080 : 0, (s << 3) in each of the four bytes}
// (block_xor, block_add). One 8-byte LDS read per block replaces five VALU ops; the 16 entries
// occupy 32 distinct banks, so the reads of a wave never conflict.
constexpr int kBlkTblBytes = 16 * 8;
__device__ __forceinline__ void build_blk_tbl(uint2* t, uint32_t tid) {
  if (tid < 16) t[tid] = uint2{block_xor(tid), block_add(tid)};
}

// The eight table reads of MFMA step MSTEP (blocks 2m, 2m+1) and what the finish needs of the two
// blocks: NS = 4, their sign masks and exponent adds read from the block table btbl (sx = {xor
// 2m, add 2m, xor 2m+1, add 2m+1}: fewer VALU ops); NS = 2, their fields (sx = {field 2m, field
// 2m+1}: fewer registers held until the finish). Block fields: bits 0-2 exponent add s, 3 sign,
// 4 rotation, 5 variant. The codebook table is the rotated one (both halves of each entry; field
// bits 4-5 select the table).
template <int KC, int MSTEP, bool ROT = true, int NS>
__device__ __forceinline__ void lut_lookup(const Unit& u, const uint8_t* lds, const uint8_t* btbl,
                                           uint32_t copy4, uint32_t (&raw)[8], uint32_t (&sx)[NS]) {
  static_assert(ROT, "the finish applies no rotation: the rotated tables are required");
  static_assert(NS == 2 || NS == 4, "");
  const uint32_t fb0 = stream_bits<3>(u.f, 12 * MSTEP, 6);
  const uint32_t fb1 = stream_bits<3>(u.f, 12 * MSTEP + 6, 6);
  const uint32_t vb0 = (((fb0 >> 4) & 3u) << Lut<KC>::kVarSh) | copy4;
  const uint32_t vb1 = (((fb1 >> 4) & 3u) << Lut<KC>::kVarSh) | copy4;
  constexpr int I = 8 * MSTEP;
  raw[0] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 0>(u.c, vb0));
  raw[1] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 1>(u.c, vb0));
  raw[2] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 2>(u.c, vb0));
  raw[3] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 3>(u.c, vb0));
  raw[4] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 4>(u.c, vb1));
  raw[5] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 5>(u.c, vb1));
  raw[6] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 6>(u.c, vb1));
  raw[7] = *reinterpret_cast<const uint32_t*>(lds + code_addr<KC, I + 7>(u.c, vb1));
  if constexpr (NS == 4) {
    const uint2 t0 = *reinterpret_cast<const uint2*>(btbl + ((fb0 << 3) & 0x78u));
    const uint2 t1 = *reinterpret_cast<const uint2*>(btbl + ((fb1 << 3) & 0x78u));
    sx[0] = t0.x; sx[1] = t0.y; sx[2] = t1.x; sx[3] = t1.y;
  } else {
    sx[0] = fb0;
    sx[1] = fb1;
  }
}

// A fragment from the table reads: sign flip, exponent add, one v_xad per dword
// (src/gpu/expert_kernel.hip:594-617; the rotation, src/quant/blockquant.cpp:826-828, is in the
// table).
template <int NS>
__device__ __forceinline__ v8i lut_finish(const uint32_t (&raw)[8], const uint32_t (&sx)[NS]) {
  v8i a;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint32_t xm = NS == 4 ? sx[2 * b] : block_xor(sx[b % NS]);
    const uint32_t ad = NS == 4 ? sx[(2 * b + 1) % NS] : block_add(sx[b % NS]);
#pragma unroll
    for (int i = 0; i < 4; ++i) a[4 * b + i] = (int)((raw[4 * b + i] ^ xm) + ad);
  }
  return a;
}

template <int KC, bool ROT = true, int NS>
__device__ __forceinline__ void lut_lookup_step(const Unit& u, const uint8_t* lds, const uint8_t* btbl,
                                                uint32_t copy4, int m, uint32_t (&raw)[8], uint32_t (&sx)[NS]) {
  switch (m) {
    case 0: lut_lookup<KC, 0, ROT>(u, lds, btbl, copy4, raw, sx); break;
    case 1: lut_lookup<KC, 1, ROT>(u, lds, btbl, copy4, raw, sx); break;
    case 2: lut_lookup<KC, 2, ROT>(u, lds, btbl, copy4, raw, sx); break;
    case 3: lut_lookup<KC, 3, ROT>(u, lds, btbl, copy4, raw, sx); break;
    case 4: lut_lookup<KC, 4, ROT>(u, lds, btbl, copy4, raw, sx); break;
    case 5: lut_lookup<KC, 5, ROT>(u, lds, btbl, copy4, raw, sx); break;
    case 6: lut_lookup<KC, 6, ROT>(u, lds, btbl, copy4, raw, sx); break;
    default: lut_lookup<KC, 7, ROT>(u, lds, btbl, copy4, raw, sx); break;
  }
}

// Makes opaque, at the top of MFMA step MSTEP, only the registers that step reads (the code
// dwords of codes 8m..8m+7 with their alignbit neighbours, the field dwords of blocks 2m, 2m+1):
// the step's extraction cannot be hoisted above it, and the step waits only for the load chunks
// it needs (chunk j = code dwords 4j..4j+3; loads complete in issue order).
template <int MSTEP>
__device__ __forceinline__ void pin_step(Unit& u) {
  constexpr int k0 = (80 * MSTEP - 6) < 0 ? 0 : (80 * MSTEP - 6) >> 5;
  constexpr int k1 = (80 * MSTEP + 79) >> 5 > 19 ? 19 : (80 * MSTEP + 79) >> 5;
#pragma unroll
  for (int k = k0; k <= k1; ++k) AFFX_PIN(u.c[k]);
  AFFX_PIN(u.f[(12 * MSTEP) >> 5]);
  if constexpr (((12 * MSTEP + 11) >> 5) != ((12 * MSTEP) >> 5)) AFFX_PIN(u.f[(12 * MSTEP + 11) >> 5]);
}

__device__ __forceinline__ void pin_step(Unit& u, int m) {
  switch (m) {
    case 0: pin_step<0>(u); break;
    case 1: pin_step<1>(u); break;
    case 2: pin_step<2>(u); break;
    case 3: pin_step<3>(u); break;
    case 4: pin_step<4>(u); break;
    case 5: pin_step<5>(u); break;
    case 6: pin_step<6>(u); break;
    default: pin_step<7>(u); break;
  }
}

// One unit, fields first, then the code chunks in order.
__device__ __forceinline__ void load_unit_ordered(Unit& u, const uint8_t* codes, const uint8_t* fields,
                                                  uint64_t tile, uint32_t lane) {
  const uint32_t* fp = reinterpret_cast<const uint32_t*>(fields + tile * kTileFieldBytes + lane * 12);
  u.f[0] = __builtin_nontemporal_load(fp);
  u.f[1] = __builtin_nontemporal_load(fp + 1);
  u.f[2] = __builtin_nontemporal_load(fp + 2);
  __builtin_amdgcn_sched_barrier(0);
  const uint8_t* cp = codes + tile * kTileCodeBytes + lane * 16;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cp + j * 1024));
    u.c[4 * j] = v[0]; u.c[4 * j + 1] = v[1]; u.c[4 * j + 2] = v[2]; u.c[4 * j + 3] = v[3];
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Three E4M3 terms of four values (|v| < 256) with the hardware conversion (round to nearest
// even, identical to f32_to_e4m3 in this range): returns the packed bytes of each term.
__device__ __forceinline__ void split3x4(float v0, float v1, float v2, float v3, uint32_t& q0,
                                         uint32_t& q1, uint32_t& q2) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  uint32_t t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, (int)t, true);
  q0 = t;
  v2f a = __builtin_amdgcn_cvt_pk_f32_fp8((int)t, false), b = __builtin_amdgcn_cvt_pk_f32_fp8((int)t, true);
  v0 = (v0 - a.x) * 16.0f; v1 = (v1 - a.y) * 16.0f; v2 = (v2 - b.x) * 16.0f; v3 = (v3 - b.y) * 16.0f;
  t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, (int)t, true);
  q1 = t;
  a = __builtin_amdgcn_cvt_pk_f32_fp8((int)t, false);
  b = __builtin_amdgcn_cvt_pk_f32_fp8((int)t, true);
  v0 = (v0 - a.x) * 16.0f; v1 = (v1 - a.y) * 16.0f; v2 = (v2 - b.x) * 16.0f; v3 = (v3 - b.y) * 16.0f;
  t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, (int)t, true);
  q2 = t;
}

// The same for two values: returns the two bytes of each term in bits 0-15.
__device__ __forceinline__ void split3x2(float v0, float v1, uint32_t& q0, uint32_t& q1, uint32_t& q2) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  uint32_t t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  q0 = t & 0xFFFFu;
  v2f a = __builtin_amdgcn_cvt_pk_f32_fp8((int)t, false);
  v0 = (v0 - a.x) * 16.0f; v1 = (v1 - a.y) * 16.0f;
  t = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  q1 = t & 0xFFFFu;
  a = __builtin_amdgcn_cvt_pk_f32_fp8((int)t, false);
  v0 = (v0 - a.x) * 16.0f; v1 = (v1 - a.y) * 16.0f;
  q2 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false) & 0xFFFFu;
}

// ------------------------------------------------------------------------------------------------
// K order of the B rows
// ------------------------------------------------------------------------------------------------
// The routed GEMM's activation rows (x terms for gate/up, SwiGLU terms for down) are stored in
// MFMA-step order: column col = 1024 s + 256 kg + 32 m + i (super-step s, lane group kg, step m,
// i < 32) sits at byte (8 s + m) * 128 + 32 kg + i, so the 128 bytes one MFMA step needs from a
// row are one run.
__host__ __device__ inline uint32_t kperm(uint32_t col) {
  return ((col >> 10) * 8u + ((col >> 5) & 7u)) * 128u + ((col >> 8) & 3u) * 32u + (col & 31u);
}

// One token's bf16 row x (+ the low part xlo, or null): its exponent sigma (returned: the row's
// largest magnitude times 2^sigma lies in [128, 256)) and tx (2 or 3) E4M3 terms of every element
// times 2^sigma, term j at row + j * hidden + pos(col), pos = kperm (KPERM) or the identity. All
// 256 threads of the workgroup call it (red: 4 floats of LDS). x, xlo 16-byte aligned; hidden a
// multiple of 8, at most 8192.
template <bool KPERM>
__device__ __forceinline__ int row_terms(const uint16_t* __restrict__ x, const uint16_t* __restrict__ xlo,
                                         uint32_t hidden, uint32_t tx, uint8_t* __restrict__ row, float* red) {
  // thread tid holds the 8-element chunks tid + 256 i (at most 4), loaded once
  constexpr int kMaxChunks = 4;
  const uint32_t tid = threadIdx.x, nch = hidden / 8;
  const uint4* xr = reinterpret_cast<const uint4*>(x);
  const uint4* lr = reinterpret_cast<const uint4*>(xlo);
  uint4 hv[kMaxChunks], lv[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const uint32_t ch = tid + 256u * i;
    hv[i] = ch < nch ? xr[ch] : uint4{0u, 0u, 0u, 0u};
    lv[i] = (lr && ch < nch) ? lr[ch] : uint4{0u, 0u, 0u, 0u};
  }
  float v[kMaxChunks][8];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const uint32_t hw[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w}, lw[4] = {lv[i].x, lv[i].y, lv[i].z, lv[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[i][2 * k] = __uint_as_float(hw[k] << 16) + __uint_as_float(lw[k] << 16);
      v[i][2 * k + 1] = __uint_as_float(hw[k] & 0xFFFF0000u) + __uint_as_float(lw[k] & 0xFFFF0000u);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[i][k]));
  }
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int sigma = amax > 0.f ? 7 - ilogbf(amax) : 0;
  // E4M3 terms, 8 bytes per term and chunk (8 consecutive columns stay consecutive in step order)
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const uint32_t ch = tid + 256u * i;
    if (ch < nch) {
      uint32_t a0, a1, a2, b0, b1, b2;
      split3x4(ldexpf(v[i][0], sigma), ldexpf(v[i][1], sigma), ldexpf(v[i][2], sigma), ldexpf(v[i][3], sigma),
               a0, a1, a2);
      split3x4(ldexpf(v[i][4], sigma), ldexpf(v[i][5], sigma), ldexpf(v[i][6], sigma), ldexpf(v[i][7], sigma),
               b0, b1, b2);
      uint8_t* dst = row + (KPERM ? kperm(8 * ch) : 8 * ch);
      *reinterpret_cast<uint2*>(dst) = uint2{a0, b0};
      *reinterpret_cast<uint2*>(dst + hidden) = uint2{a1, b1};
      if (tx == 3) *reinterpret_cast<uint2*>(dst + 2 * (uint64_t)hidden) = uint2{a2, b2};
    }
  }
  return sigma;
}

// Calls f(IConst<I>{}) for I = B .. E-1: a loop whose index is a compile-time constant in the body.
template <int N>
struct IConst {
  static constexpr int value = N;
};
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(IConst<B>{});
    static_for<B + 1, E>(f);
  }
}

}  // namespace affx
