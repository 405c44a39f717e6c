// CPU emulation of the HIP surface libaffx's kernels use (test infrastructure, never shipped).
//
// A kernel launch runs one workgroup at a time with one std::thread per work-item (launches with
// dynamic LDS run all their workgroups at once instead, each with its own LDS block, as a kernel
// that synchronises across workgroups needs them co-resident); __syncthreads
// is a real block barrier and every cross-lane operation (shuffles, ballot, the MFMA) exchanges
// values through per-wave slots between two wave barriers. Device memory is ordinary host memory,
// so building with -fsanitize=address turns any out-of-bounds access of a kernel into an ASan
// report on the CPU. The fp8 MFMA is computed exactly (double accumulation) with the gfx950 lane
// layout the kernels assume (A/B lane l = row/column l%16 and k-group l/16, D lane l element v =
// D[4*(l/16)+v][l%16]); tests/test_gpu_decode.py pins that layout on the hardware.
#pragma once
#include <barrier>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>
#include <algorithm>
#include <atomic>
#include <mutex>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define AFFX_PIN(x) ((void)0)  // (the library's register pin is device assembly)
#define __launch_bounds__(...)
#define __restrict__
#define __shared__ static
#define __align__(x) __attribute__((aligned(x)))

struct emu_dim3 { uint32_t x = 1, y = 1, z = 1; };
struct dim3 { uint32_t x, y, z; dim3(uint32_t a = 1, uint32_t b = 1, uint32_t c = 1) : x(a), y(b), z(c) {} };
extern thread_local emu_dim3 threadIdx, blockIdx;
extern emu_dim3 blockDim, gridDim;

typedef int hipError_t;
typedef void* hipStream_t;
#define hipSuccess 0
inline const char* hipGetErrorString(int) { return "emu"; }
inline int hipGetLastError() { return 0; }
inline int hipGetDevice(int* d) { *d = 0; return 0; }
struct hipDeviceProp_t { char gcnArchName[64]; int multiProcessorCount; };
inline int hipGetDeviceProperties(hipDeviceProp_t* p, int) { strcpy(p->gcnArchName, "gfx950"); p->multiProcessorCount = 256; return 0; }
inline int hipMemsetAsync(void* p, int v, size_t n, hipStream_t) { memset(p, v, n); return 0; }
enum hipMemcpyKind { hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2, hipMemcpyDeviceToDevice = 3 };
inline int hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) { memmove(d, s, n); return 0; }
inline int hipStreamSynchronize(hipStream_t) { return 0; }  // launches run to completion
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
inline int hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* st) { *st = hipStreamCaptureStatusNone; return 0; }
#define HIP_SYMBOL(x) (&(x))
inline int hipGetSymbolAddress(void** p, const void* sym) { *p = const_cast<void*>(sym); return 0; }
// device shape of the emulation: AFFX_EMU_CUS compute units (default 4), one resident workgroup each
inline int emu_cus() { const char* e = getenv("AFFX_EMU_CUS"); return e ? atoi(e) : 4; }
enum { hipDeviceAttributeMultiprocessorCount = 1, hipFuncAttributeMaxDynamicSharedMemorySize = 2 };
inline int hipDeviceGetAttribute(int* v, int attr, int) { *v = attr == hipDeviceAttributeMultiprocessorCount ? emu_cus() : 0; return 0; }
inline int hipFuncSetAttribute(const void*, int, int) { return 0; }
inline int hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, const void*, int, size_t) { *n = 1; return 0; }

struct uint2 { uint32_t x, y; };
struct uint4 { uint32_t x, y, z, w; };
struct float4 { float x, y, z, w; };
inline uint4 make_uint4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return {a, b, c, d}; }
inline float4 make_float4(float a, float b, float c, float d) { return {a, b, c, d}; }

inline float __uint_as_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
inline uint32_t __float_as_uint(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; memcpy(&f, &u, 4); return f; }
inline int __float_as_int(float f) { int u; memcpy(&u, &f, 4); return u; }
inline int __popc(uint32_t v) { return __builtin_popcount(v); }
inline int __popcll(uint64_t v) { return __builtin_popcountll(v); }
inline float __fsub_rn(float a, float b) { volatile float r = a - b; return r; }
inline float __fadd_rn(float a, float b) { volatile float r = a + b; return r; }
inline float __fmul_rn(float a, float b) { volatile float r = a * b; return r; }
inline float __fdiv_rn(float a, float b) { volatile float r = a / b; return r; }
inline double __dmul_rn(double a, double b) { volatile double r = a * b; return r; }
inline double __ddiv_rn(double a, double b) { volatile double r = a / b; return r; }

// v_exp_f32 / v_rcp_f32: the library uses them where a few ulp are within its tolerance
inline float __builtin_amdgcn_exp2f(float x) { return exp2f(x); }
inline float __builtin_amdgcn_rcpf(float x) { return 1.0f / x; }
inline uint32_t __builtin_amdgcn_alignbit(uint32_t hi, uint32_t lo, uint32_t s) {
  return (uint32_t)((((uint64_t)hi << 32) | lo) >> (s & 31));
}
inline uint32_t __builtin_amdgcn_perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  uint8_t bytes[8];
  for (int i = 0; i < 4; ++i) { bytes[i] = (s1 >> (8 * i)) & 0xff; bytes[4 + i] = (s0 >> (8 * i)) & 0xff; }
  uint32_t out = 0;
  for (int i = 0; i < 4; ++i) {
    uint32_t sb = (sel >> (8 * i)) & 0xff, v;
    if (sb < 8) v = bytes[sb]; else if (sb == 12) v = 0; else if (sb >= 13) v = 0xff; else { fprintf(stderr, "perm sel\n"); abort(); }
    out |= v << (8 * i);
  }
  return out;
}
#define __builtin_amdgcn_sched_barrier(x) ((void)0)
#define __builtin_amdgcn_sched_group_barrier(m, n, id) ((void)0)
#define __builtin_amdgcn_s_sleep(x) std::this_thread::yield()
#define __builtin_amdgcn_s_setprio(x) ((void)0)
#define __builtin_amdgcn_s_waitcnt(x) std::atomic_thread_fence(std::memory_order_seq_cst)
// __hip_atomic_* are clang builtins on the host too; their scope constants are clang's
#ifndef __HIP_MEMORY_SCOPE_AGENT
#define __HIP_MEMORY_SCOPE_AGENT 4
#endif
#ifndef __HIP_MEMORY_SCOPE_WORKGROUP
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#endif
#define __builtin_amdgcn_fence(order, scope) std::atomic_thread_fence(std::memory_order_seq_cst)
template <typename T> inline T __builtin_amdgcn_readfirstlane(T v) { return v; }  // callers pass uniform values
#define __builtin_nontemporal_load(p) (*(p))

// ---- wave / block synchronisation ----
struct EmuBlock {
  std::barrier<>* block_bar;
  std::barrier<>* wave_bar[16];
  uint8_t* lds;                // dynamic LDS of the block (concurrent launches)
  uint64_t xfer[16][64][16];   // per-wave lane exchange (up to 16 x 32-bit words... in 64-bit slots)
};
extern thread_local EmuBlock* emu_blk;
inline void __syncthreads() { emu_blk->block_bar->arrive_and_wait(); }
inline void __builtin_amdgcn_s_barrier() { __syncthreads(); }
inline uint32_t emu_lane() { return threadIdx.x & 63; }
inline uint32_t emu_wave() { return threadIdx.x >> 6; }
// v_mbcnt_lo/hi: add the count of set mask bits below this lane (lanes 0-31 / 32-63)
inline uint32_t __builtin_amdgcn_mbcnt_lo(uint32_t mask, uint32_t add) {
  const uint32_t l = emu_lane() < 32 ? emu_lane() : 32;
  return add + (uint32_t)__builtin_popcount(l >= 32 ? mask : mask & ((1u << l) - 1u));
}
inline uint32_t __builtin_amdgcn_mbcnt_hi(uint32_t mask, uint32_t add) {
  const uint32_t l = emu_lane() > 32 ? emu_lane() - 32 : 0;
  return add + (uint32_t)__builtin_popcount(mask & ((1u << l) - 1u));
}
inline void emu_wave_sync() { emu_blk->wave_bar[emu_wave()]->arrive_and_wait(); }
#define __builtin_amdgcn_wave_barrier() emu_wave_sync()
#define AFFX_DYN_LDS(name) uint8_t* name = emu_blk->lds

template <typename T>
inline T emu_exchange(T v, uint32_t src) {
  static_assert(sizeof(T) <= 8, "");
  uint64_t bits = 0; memcpy(&bits, &v, sizeof(T));
  emu_blk->xfer[emu_wave()][emu_lane()][0] = bits;
  emu_wave_sync();
  uint64_t got = emu_blk->xfer[emu_wave()][src & 63][0];
  emu_wave_sync();
  T r; memcpy(&r, &got, sizeof(T)); return r;
}
template <typename T> inline T __shfl_xor(T v, int o, int width = 64) { return emu_exchange(v, emu_lane() ^ o); }
template <typename T> inline T __shfl(T v, int src, int width = 64) { return emu_exchange(v, (uint32_t)src & 63u); }
template <typename T> inline T __builtin_amdgcn_readlane(T v, uint32_t l) { return emu_exchange(v, l); }
inline int __builtin_amdgcn_ds_bpermute(int addr, int v) { return emu_exchange(v, ((uint32_t)addr >> 2) & 63); }
template <typename T> inline T __shfl_down(T v, int d, int width = 64) {
  uint32_t l = emu_lane(); uint32_t src = ((l % width) + d < (uint32_t)width) ? l + d : l;
  return emu_exchange(v, src);
}
template <typename T> inline T __shfl_up(T v, int d, int width = 64) {
  uint32_t l = emu_lane(); uint32_t src = (l % width) >= (uint32_t)d ? l - d : l;
  return emu_exchange(v, src);
}
// DPP row shifts (dpp_ctrl 0x101-0x10F row_shl, 0x111-0x11F row_shr; rows of 16 lanes) and quad
// permutes (0x00-0xFF: lane 4q + i reads lane 4q + ((ctrl >> 2i) & 3))
inline int __builtin_amdgcn_update_dpp(int old, int src, int ctrl, int, int, bool bound_ctrl) {
  const uint32_t l = emu_lane(), rl = l & 15;
  int from = -1;
  if (ctrl >= 0x101 && ctrl <= 0x10F && rl + (ctrl - 0x100) < 16) from = (int)l + (ctrl - 0x100);
  if (ctrl >= 0x111 && ctrl <= 0x11F && (int)rl - (ctrl - 0x110) >= 0) from = (int)l - (ctrl - 0x110);
  if (ctrl >= 0 && ctrl <= 0xFF) from = (int)((l & ~3u) | ((uint32_t)(ctrl >> (2 * (l & 3))) & 3u));  // quad_perm
  const int v = emu_exchange(src, from < 0 ? l : (uint32_t)from);
  return from < 0 ? (bound_ctrl ? 0 : old) : v;
}
inline uint64_t __ballot(int pred) {
  emu_blk->xfer[emu_wave()][emu_lane()][0] = pred ? 1 : 0;
  emu_wave_sync();
  uint64_t m = 0;
  for (int i = 0; i < 64; ++i) if (emu_blk->xfer[emu_wave()][i][0]) m |= 1ull << i;
  emu_wave_sync();
  return m;
}
inline uint32_t atomicOr(uint32_t* p, uint32_t v) { return __atomic_fetch_or(p, v, __ATOMIC_SEQ_CST); }
inline uint32_t atomicAdd(uint32_t* p, uint32_t v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline uint32_t atomicMin(uint32_t* p, uint32_t v) {
  uint32_t cur = __atomic_load_n(p, __ATOMIC_SEQ_CST);
  while (v < cur && !__atomic_compare_exchange_n(p, &cur, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST)) {
  }
  return cur;
}
inline uint32_t min(uint32_t a, uint32_t b) { return a < b ? a : b; }

// ---- buffer resources and direct global->LDS loads ----
// A raw buffer resource is a base and a byte count; a read past the count returns zeros, as on
// the device. A direct-to-LDS load writes lane l's `size` bytes at lds + off + l * size.
struct emu_rsrc { const uint8_t* base; uint32_t n; };
#define __amdgpu_buffer_rsrc_t emu_rsrc
inline emu_rsrc __builtin_amdgcn_make_buffer_rsrc(void* p, short, int n, int) { return {(const uint8_t*)p, (uint32_t)n}; }
template <typename T> inline T emu_buf_load(emu_rsrc r, uint32_t voff, uint32_t soff) {
  T v;
  const uint64_t o = (uint64_t)voff + soff;
  if (o + sizeof(T) > r.n) { memset(&v, 0, sizeof(T)); return v; }
  memcpy(&v, r.base + o, sizeof(T));
  return v;
}
typedef uint32_t emu_u32x4 __attribute__((ext_vector_type(4)));
inline uint8_t __builtin_amdgcn_raw_buffer_load_b8(emu_rsrc r, uint32_t v, uint32_t s, int) { return emu_buf_load<uint8_t>(r, v, s); }
inline uint32_t __builtin_amdgcn_raw_buffer_load_b32(emu_rsrc r, uint32_t v, uint32_t s, int) { return emu_buf_load<uint32_t>(r, v, s); }
inline emu_u32x4 __builtin_amdgcn_raw_buffer_load_b128(emu_rsrc r, uint32_t v, uint32_t s, int) { return emu_buf_load<emu_u32x4>(r, v, s); }
template <typename T> inline void emu_buf_store(T v, emu_rsrc r, uint32_t voff, uint32_t soff) {
  const uint64_t o = (uint64_t)voff + soff;
  if (o + sizeof(T) > r.n) return;  // past the range: dropped, as on the device
  memcpy(const_cast<uint8_t*>(r.base) + o, &v, sizeof(T));
}
inline void __builtin_amdgcn_raw_buffer_store_b128(emu_u32x4 v, emu_rsrc r, uint32_t vo, uint32_t so, int) { emu_buf_store(v, r, vo, so); }
inline void __builtin_amdgcn_raw_ptr_buffer_load_lds(emu_rsrc r, void* lds, int size, uint32_t v, uint32_t s, int off, int) {
  const uint64_t o = (uint64_t)v + s;
  uint8_t* dst = (uint8_t*)lds + off + (threadIdx.x & 63) * size;
  if (o + size > r.n) memset(dst, 0, size); else memcpy(dst, r.base + o, size);
}
#define AFFX_LDS_PTR(p) ((void*)(p))
inline void __builtin_amdgcn_s_barrier();

// ---- MFMA 16x16x128 fp8 x fp8 -> f32, lane layout as on gfx950 ----
typedef int emu_v8i __attribute__((ext_vector_type(8)));
typedef float emu_v4f __attribute__((ext_vector_type(4)));
inline float emu_e4m3(uint32_t b) {
  const int s = (b >> 7) & 1, e = (b >> 3) & 15, m = b & 7;
  float f = e == 0 ? ldexpf(m / 8.0f, -6) : (e == 15 && m == 7 ? NAN : ldexpf(1.0f + m / 8.0f, e - 7));
  return s ? -f : f;
}
// hardware f32 -> E4M3 (OCP) conversion, round to nearest even, for the in-range values kernels
// pass (|v| <= 448, the largest finite E4M3)
inline uint32_t emu_to_e4m3(float v) {
  const uint32_t s = (__float_as_uint(v) >> 24) & 0x80u;
  const float a = fabsf(v);
  if (!(a <= 448.f)) { fprintf(stderr, "cvt_pk_fp8_f32: out of range %g\n", v); abort(); }
  if (a < 0.015625f) return s | (uint32_t)rintf(a * 512.0f);
  const uint32_t au = __float_as_uint(a);
  int e = (int)(au >> 23) - 127;
  uint32_t m3 = (au >> 20) & 7u;
  const uint32_t rem = au & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) { if (++m3 == 8u) { m3 = 0; ++e; } }
  return s | ((uint32_t)(e + 7) << 3) | m3;
}
inline int __builtin_amdgcn_cvt_pk_fp8_f32(float a, float b, int old, bool hi) {
  const uint32_t pair = emu_to_e4m3(a) | (emu_to_e4m3(b) << 8);
  return (int)(hi ? (((uint32_t)old & 0xFFFFu) | (pair << 16)) : (((uint32_t)old & 0xFFFF0000u) | pair));
}
typedef float emu_v2f __attribute__((ext_vector_type(2)));
inline emu_v2f __builtin_amdgcn_cvt_pk_f32_fp8(int w, bool hi) {
  const uint32_t u = (uint32_t)w >> (hi ? 16 : 0);
  emu_v2f r;
  r.x = emu_e4m3(u & 0xFF);
  r.y = emu_e4m3((u >> 8) & 0xFF);
  return r;
}

// Scales: lane l's E8M0 byte (selected by opsel) multiplies its own 32 K values, row l % 16 of A or
// column l % 16 of B in K group l / 16 (the layout checked on gfx950).
inline emu_v4f __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(emu_v8i a, emu_v8i b, emu_v4f c, int, int, int opa,
                                                                int sa, int opb, int sb) {
  uint32_t w = emu_wave(), l = emu_lane();
  for (int i = 0; i < 8; ++i) emu_blk->xfer[w][l][i] = (uint32_t)a[i] | ((uint64_t)(uint32_t)b[i] << 32);
  emu_blk->xfer[w][l][8] = (((uint32_t)sa >> (8 * opa)) & 0xff) | ((uint64_t)(((uint32_t)sb >> (8 * opb)) & 0xff) << 32);
  emu_wave_sync();
  emu_v4f d = c;
  for (int v = 0; v < 4; ++v) {
    const uint32_t row = 4 * (l / 16) + v, col = l % 16;
    double acc = 0;
    for (int g = 0; g < 4; ++g) {
      double part = 0;
      for (int i = 0; i < 8; ++i) {
        uint32_t A = (uint32_t)emu_blk->xfer[w][row + 16 * g][i], B = (uint32_t)(emu_blk->xfer[w][col + 16 * g][i] >> 32);
        for (int p = 0; p < 4; ++p) part += (double)emu_e4m3((A >> (8 * p)) & 0xff) * emu_e4m3((B >> (8 * p)) & 0xff);
      }
      const int ea = (int)(emu_blk->xfer[w][row + 16 * g][8] & 0xff), eb = (int)(emu_blk->xfer[w][col + 16 * g][8] >> 32);
      acc += ldexp(part, ea + eb - 254);
    }
    d[v] = c[v] + (float)acc;
  }
  emu_wave_sync();
  return d;
}

// ---- launch ----
// Sequential: one block at a time, blockDim.x threads created once per launch.
template <typename F, typename... Args>
void emu_launch_seq(F kernel, dim3 grid, dim3 block, Args... args) {
  gridDim = {grid.x, grid.y, grid.z};
  blockDim = {block.x, block.y, block.z};
  const uint32_t nt = block.x;
  const uint64_t nblocks = (uint64_t)grid.x * grid.y * grid.z;
  std::barrier<> start(nt + 1), done(nt + 1), bb(nt);
  EmuBlock blk;
  blk.block_bar = &bb;
  blk.lds = nullptr;
  std::vector<std::barrier<>*> wbs;
  for (uint32_t w = 0; w < (nt + 63) / 64; ++w) {
    wbs.push_back(new std::barrier<>(std::min<uint32_t>(64, nt - 64 * w)));
    blk.wave_bar[w] = wbs.back();
  }
  std::vector<std::thread> ts;
  for (uint32_t t = 0; t < nt; ++t)
    ts.emplace_back([&, t]() {
      emu_blk = &blk;
      for (uint64_t b = 0; b < nblocks; ++b) {
        start.arrive_and_wait();
        threadIdx = {t, 0, 0};
        blockIdx = {(uint32_t)(b % grid.x), (uint32_t)((b / grid.x) % grid.y), (uint32_t)(b / ((uint64_t)grid.x * grid.y))};
        kernel(args...);
        done.arrive_and_wait();
      }
    });
  for (uint64_t b = 0; b < nblocks; ++b) {
    start.arrive_and_wait();
    done.arrive_and_wait();
  }
  for (auto& th : ts) th.join();
  for (auto* w : wbs) delete w;
}

// Concurrent: every block at once (1-D grids), each with its own barriers and `shm` bytes of
// dynamic LDS allocated as a separate heap block (ASan sees any access past it).
template <typename F, typename... Args>
void emu_launch_all(F kernel, dim3 grid, size_t shm, dim3 block, Args... args) {
  gridDim = {grid.x, grid.y, grid.z};
  blockDim = {block.x, block.y, block.z};
  const uint32_t nt = block.x, nb = grid.x;
  if (grid.y != 1 || grid.z != 1) { fprintf(stderr, "concurrent launch needs a 1-D grid\n"); abort(); }
  std::vector<EmuBlock> blks(nb);
  std::vector<std::barrier<>*> owned;
  for (uint32_t b = 0; b < nb; ++b) {
    owned.push_back(new std::barrier<>(nt));
    blks[b].block_bar = owned.back();
    for (uint32_t w = 0; w < (nt + 63) / 64; ++w) {
      owned.push_back(new std::barrier<>(std::min<uint32_t>(64, nt - 64 * w)));
      blks[b].wave_bar[w] = owned.back();
    }
    blks[b].lds = new uint8_t[shm];
    memset(blks[b].lds, 0xA5, shm);  // LDS starts undefined on the device
  }
  // at most emu_cus() workgroups at a time, as many as the emulated device holds: every grid
  // that needs its workgroups co-resident is sized to that, and larger grids run in waves
  const uint32_t chunk = (uint32_t)std::max(1, emu_cus());
  for (uint32_t b0 = 0; b0 < nb; b0 += chunk) {
    std::vector<std::thread> ts;
    for (uint32_t b = b0; b < nb && b < b0 + chunk; ++b)
      for (uint32_t t = 0; t < nt; ++t)
        ts.emplace_back([&, b, t]() {
          emu_blk = &blks[b];
          threadIdx = {t, 0, 0};
          blockIdx = {b, 0, 0};
          kernel(args...);
        });
    for (auto& th : ts) th.join();
  }
  for (auto& bl : blks) delete[] bl.lds;
  for (auto* p : owned) delete p;
}

template <typename F, typename... Args>
void emu_launch(F kernel, dim3 grid, dim3 block, size_t shm, Args... args) {
  if (shm) emu_launch_all(kernel, grid, shm, block, args...);
  else emu_launch_seq(kernel, grid, block, args...);
}
#define hipLaunchKernelGGL(k, g, b, shm, s, ...) emu_launch(k, dim3(g), dim3(b), (size_t)(shm), __VA_ARGS__)
