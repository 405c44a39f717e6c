// The codebook producer on the GPU: sample collection, the joint fit of the 2 x 1024 quad
// codebook (k-means++ seeding, Lloyd passes, an octave-seeded second variant, block-level EM),
// and its E4M3 projection, packing and unpacking. The quad format only: 4-wide codes, 1024
// entries, 2 variants, power-of-two block scales (src/quant/blockquant.cpp:75-86, 155-166,
// 203-492). aff-quantize runs these once per container before it quantises
// (tools/aff_quantize.cpp:402-434); each result equals the reference CPU path's bit for bit.
//
// The reference's floating-point results depend on summation order in three places; each is
// kept as such:
//  * a k-means++ draw compares a running double sum of d2 with a fraction of their double total
//    (blockquant.cpp:284-290). Here the sums are parallel, and a pick is taken only where the
//    rounding-error bound of any summation order (the reference's sequential one included)
//    cannot move it. Otherwise one wave repeats the reference's sequential sums exactly (rare:
//    the bound is about n * 2^-53 of the total, a draw's step is about 1/n of it).
//  * a Lloyd centroid is a double sum over its items in item order (blockquant.cpp:222-233): the
//    items are sorted by centroid with a stable counting sort, then one thread per centroid adds
//    its run in order.
//  * the convergence shift and the reseed gap are sequential double sums, added by one thread
//    in the reference's order.
// Distances are float (nearest entry) or double (k-means++), one rounding per operation in the
// reference's order; the reference builds its CPU path without contraction, and so does this
// file.
#include <cfloat>
#include <cmath>

#include "affx_common.h"

#pragma clang fp contract(off)

namespace affx {
namespace {

constexpr uint32_t kFitK = kLut;                       // entries per variant
constexpr uint32_t kCbFloats = kVariants * kLut * 4;   // 8192 floats, [variant][entry][4]
constexpr uint32_t kEmRounds = 12;                     // blockquant.cpp:341
constexpr uint32_t kEmIters = 6;                       // Lloyd passes per variant and round
constexpr uint32_t kKppThreads = 256, kKppPer = 16;
constexpr uint32_t kKppChunk = kKppThreads * kKppPer;  // items per d2-update workgroup
constexpr uint32_t kPickThreads = kKppChunk / 4;       // the pick scans one chunk, 4 items a thread
constexpr uint32_t kSortSteps = 32;                    // 64-key steps per counting-sort wave
constexpr uint32_t kSortChunk = 64 * kSortSteps;      // keys per counting-sort wave
constexpr uint32_t kAssignThreads = 256;
constexpr uint32_t kSeqBuf = 512;                      // doubles staged per step of a sequential sum

// Device state of a fit, at the start of the workspace.
struct FitState {
  uint32_t pick_ok;     // the current k-means++ pick was written by the certified path
  uint32_t lloyd_done;  // the current refit converged (shift < 1e-7)
  uint32_t em_active;   // the current EM round runs
  uint32_t em_stop;     // member counts repeated: no further round
  uint64_t nm[2];       // member blocks of each variant this round
  uint64_t prev[2];     // ... the round before
  uint64_t n_seq_picks; // k-means++ picks taken by the sequential path
  uint64_t n_passes;    // Lloyd passes run
  double gap;           // reseed offset scale (blockquant.cpp:318-319), once computed
  uint32_t gap_ready;
  uint32_t pad;
};

// A pass's element list: all blocks of the fit (items 0 .. 4 n_blocks - 1), the member blocks of
// one variant (items of part[...] in order), or the blocks themselves (the EM partition).
enum PassMode : int { kAll = 0, kMember = 1, kPartition = 2 };

// Elements of a pass of this mode, 0 when the pass is skipped (converged, round inactive, no
// members).
__device__ __forceinline__ uint64_t pass_len(const FitState* st, int mode, uint32_t v, uint64_t n_blocks) {
  if (mode == kPartition) return st->em_active ? n_blocks : 0;
  if (st->lloyd_done) return 0;
  if (mode == kAll) return 4 * n_blocks;
  return st->em_active ? 4 * st->nm[v] : 0;
}

// wide_argmin (blockquant.cpp:155-166): the squared distance in float, summed from 0 over the
// four dimensions in order, the first strict minimum.
__device__ __forceinline__ uint32_t nearest_entry(const float4* cent, float4 x, float& dmin) {
  float bd = FLT_MAX;
  uint32_t best = 0;
#pragma unroll 8
  for (uint32_t c = 0; c < kFitK; ++c) {
    const float4 e = cent[c];
    const float a = e.x - x.x, b = e.y - x.y, g = e.z - x.z, h = e.w - x.w;
    float s = a * a;
    s = s + b * b;
    s = s + g * g;
    s = s + h * h;
    if (s < bd) {
      bd = s;
      best = c;
    }
  }
  dmin = bd;
  return best;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o);
  return v;
}

// Sum over a workgroup of NT threads (any order: the callers bound the error).
template <int NT>
__device__ __forceinline__ double block_sum(double v, double* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0)
    for (int w = 0; w < NT / 64; ++w) s = s + red[w];
  return s;
}

// Inclusive scan over a workgroup of NT threads through sc[NT] (Hillis-Steele); returns this
// thread's inclusive value, sc holds all of them afterwards.
template <int NT, typename T>
__device__ __forceinline__ T block_scan_incl(T v, T* sc) {
  sc[threadIdx.x] = v;
  __syncthreads();
  for (int o = 1; o < NT; o <<= 1) {
    const T add = (int)threadIdx.x >= o ? sc[threadIdx.x - o] : T(0);
    __syncthreads();
    v = v + add;
    sc[threadIdx.x] = v;
    __syncthreads();
  }
  return v;
}

// The same scan by wave: shuffle scans within each wave, then the waves' totals (one thread). The
// order of the additions differs from the LDS form; the callers bound the error either way.
template <int NT>
__device__ __forceinline__ double block_scan_incl_waves(double v, double* sc) {
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const double o = __shfl_up(v, d);
    if ((int)lane >= d) v = v + o;
  }
  __shared__ double wtot[NT / 64];
  if (lane == 63) wtot[wv] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    double run = 0.0;
    for (int w = 0; w < NT / 64; ++w) {
      run = run + wtot[w];
      wtot[w] = run;
    }
  }
  __syncthreads();
  if (wv > 0) v = v + wtot[wv - 1];
  sc[threadIdx.x] = v;
  __syncthreads();
  return v;
}

// ---- fit set-up --------------------------------------------------------------------------------

// cb = 0 but entry 0 of variant 0 = the first sample quad (blockquant.cpp:274); state cleared.
__global__ void __launch_bounds__(256) fit_init_kernel(const float* __restrict__ samples, uint64_t n_items,
                                                       float* __restrict__ cb, FitState* __restrict__ st) {
  for (uint32_t i = threadIdx.x; i < kCbFloats; i += 256) cb[i] = (i < 4 && n_items > 0) ? samples[i] : 0.0f;
  if (threadIdx.x == 0) {
    FitState s = {};
    s.prev[0] = s.prev[1] = ~0ull;
    *st = s;
  }
}

// ---- k-means++ (blockquant.cpp:270-294) --------------------------------------------------------

// d2[i] = min(d2[i], code_dist(x_i, entry c-1)) in double (blockquant.cpp:75-86, weight 1), and
// the workgroup's sum of the new d2.
__global__ void __launch_bounds__(kKppThreads) kpp_update_kernel(const float4* __restrict__ x, uint64_t n,
                                                                 const float* __restrict__ cb, uint32_t c, int first,
                                                                 double* __restrict__ d2, double* __restrict__ wgsum) {
  __shared__ double red[kKppThreads / 64];
  const float4 last = reinterpret_cast<const float4*>(cb)[c - 1];
  const double l0 = last.x, l1 = last.y, l2 = last.z, l3 = last.w;
  const uint64_t base = (uint64_t)blockIdx.x * kKppChunk + threadIdx.x;
  double sum = 0.0;
#pragma unroll 4
  for (uint32_t r = 0; r < kKppPer; ++r) {
    const uint64_t i = base + (uint64_t)r * kKppThreads;
    if (i < n) {
      const float4 v = x[i];
      const double e0 = (double)v.x - l0, e1 = (double)v.y - l1, e2 = (double)v.z - l2, e3 = (double)v.w - l3;
      double s = e0 * e0;
      s = s + e1 * e1;
      s = s + e2 * e2;
      s = s + e3 * e3;
      double cur = first ? DBL_MAX : d2[i];
      if (s < cur) cur = s;
      d2[i] = cur;
      sum = sum + cur;
    }
  }
  sum = block_sum<kKppThreads>(sum, red);
  if (threadIdx.x == 0) wgsum[blockIdx.x] = sum;
}

// The draw: the first i whose running sum of d2 reaches a * (sum of all d2), with a =
// (r % 1e6) / 1e6. Parallel prefix sums locate it; it is certified when it holds for every
// summation order within the error bound, else left to kpp_seq_kernel.
__global__ void __launch_bounds__(kPickThreads) kpp_pick_kernel(const float4* __restrict__ x, uint64_t n,
                                                                const double* __restrict__ d2,
                                                                const double* __restrict__ wgsum, uint32_t n_wg,
                                                                double a, uint32_t c, int force_seq,
                                                                float* __restrict__ cb, FitState* __restrict__ st) {
  __shared__ double sc[kPickThreads];
  __shared__ uint32_t s_w, s_i;
  __shared__ double s_pw, s_cm1, s_c0;
  const uint32_t t = threadIdx.x;
  // workgroup totals: a contiguous run per thread, then the scan over threads
  const uint32_t per = (n_wg + kPickThreads - 1) / kPickThreads;
  double run = 0.0;
  for (uint32_t j = 0; j < per; ++j) {
    const uint32_t w = t * per + j;
    if (w < n_wg) run = run + wgsum[w];
  }
  block_scan_incl_waves<kPickThreads>(run, sc);
  const double T = sc[kPickThreads - 1];
  const double aT = a * T;
  const double excl = t ? sc[t - 1] : 0.0;
  if (t == 0) {
    s_w = ~0u;
    s_i = ~0u;
  }
  __syncthreads();
  const bool finite_pos = T > 0.0 && T <= DBL_MAX;  // (uniform)
  uint32_t my_w = ~0u;
  double my_p = 0.0;
  if (finite_pos) {
    double p = excl;
    for (uint32_t j = 0; j < per; ++j) {
      const uint32_t w = t * per + j;
      if (w >= n_wg) break;
      const double q = p + wgsum[w];
      if (q >= aT) {
        my_w = w;
        my_p = p;
        break;
      }
      p = q;
    }
    if (my_w != ~0u) atomicMin(&s_w, my_w);
  }
  __syncthreads();
  if (my_w != ~0u && my_w == s_w) s_pw = my_p;
  __syncthreads();
  const uint32_t w = s_w;
  // the chunk of workgroup w: thread t holds items 4t .. 4t + 3
  double loc[4] = {0.0, 0.0, 0.0, 0.0};
  double tsum = 0.0;
  const uint64_t base = (uint64_t)(w == ~0u ? 0u : w) * kKppChunk + 4u * t;
  if (w != ~0u) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint64_t i = base + q;
      if (i < n) tsum = tsum + d2[i];
      loc[q] = tsum;
    }
  }
  block_scan_incl_waves<kPickThreads>(tsum, sc);
  const double pre = t ? sc[t - 1] : 0.0;  // the sum of the chunk's items before this thread's
  if (w != ~0u) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint64_t i = base + q;
      if (i < n && s_pw + (pre + loc[q]) >= aT) {
        atomicMin(&s_i, 4u * t + q);
        break;
      }
    }
  }
  __syncthreads();
  const uint32_t li = s_i;
  if (w != ~0u && li != ~0u) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t k = 4u * t + q;
      const double cv = s_pw + (pre + loc[q]);
      if (k == li) s_c0 = cv;
      if (k + 1 == li) s_cm1 = cv;
    }
    if (li == 0 && t == 0) s_cm1 = s_pw;
  }
  __syncthreads();
  if (t == 0) {
    bool ok = false;
    uint64_t pick = 0;
    if (T == 0.0) {
      ok = true;  // every d2 is 0: the running sum reaches 0 * total at item 0
    } else if (finite_pos && w != ~0u && li != ~0u) {
      pick = (uint64_t)w * kKppChunk + li;
      // |error| of any order of n non-negative additions <= n * 2^-53 of the exact sum, and the
      // target's product adds one rounding: margins of twice that, plus the evaluation's own.
      const double u = 0x1p-53;
      const double G = ((double)n + (double)n_wg + 256.0) * u * 1.0625;
      const double Gt = 2.0 * G + 16.0 * u;
      const bool below = pick == 0 || s_cm1 * (1.0 + Gt) < aT * (1.0 - Gt);
      const bool above = s_c0 * (1.0 - Gt) >= aT * (1.0 + Gt);
      ok = below && above && pick < n;
    }
    if (force_seq) ok = false;
    st->pick_ok = ok ? 1u : 0u;
    if (ok) {
      const float4 xv = x[pick];
      reinterpret_cast<float4*>(cb)[c] = xv;
    }
  }
}

// The reference's own sums, when the pick could not be certified: total, target, running sum,
// in item order by one lane; the wave stages the d2 through LDS.
__global__ void __launch_bounds__(64) kpp_seq_kernel(const float4* __restrict__ x, uint64_t n,
                                                     const double* __restrict__ d2, double a, uint32_t c,
                                                     float* __restrict__ cb, FitState* __restrict__ st) {
  if (st->pick_ok) return;
  __shared__ double buf[kSeqBuf];
  __shared__ uint32_t s_found;
  __shared__ uint64_t s_pick;
  const uint32_t lane = threadIdx.x;
  double tot = 0.0;
  for (uint64_t b0 = 0; b0 < n; b0 += kSeqBuf) {
    for (uint32_t j = lane; j < kSeqBuf; j += 64) buf[j] = b0 + j < n ? d2[b0 + j] : 0.0;
    __syncthreads();
    if (lane == 0) {
      const uint32_t m = (uint32_t)(n - b0 < kSeqBuf ? n - b0 : kSeqBuf);
      for (uint32_t k = 0; k < m; ++k) tot = tot + buf[k];
    }
    __syncthreads();
  }
  const double target = a * tot;
  if (lane == 0) {
    s_found = 0;
    s_pick = n - 1;
  }
  __syncthreads();
  double cum = 0.0;
  for (uint64_t b0 = 0; b0 < n; b0 += kSeqBuf) {
    for (uint32_t j = lane; j < kSeqBuf; j += 64) buf[j] = b0 + j < n ? d2[b0 + j] : 0.0;
    __syncthreads();
    if (lane == 0) {
      const uint32_t m = (uint32_t)(n - b0 < kSeqBuf ? n - b0 : kSeqBuf);
      for (uint32_t k = 0; k < m; ++k) {
        cum = cum + buf[k];
        if (cum >= target) {
          s_pick = b0 + k;
          s_found = 1;
          break;
        }
      }
    }
    __syncthreads();
    if (s_found) break;
  }
  if (lane == 0) {
    reinterpret_cast<float4*>(cb)[c] = x[s_pick];
    st->n_seq_picks += 1;
  }
}

// ---- Lloyd passes (blockquant.cpp:203-244) -----------------------------------------------------

// key[t] = nearest entry of variant v to item t of the pass.
__global__ void __launch_bounds__(kAssignThreads) lloyd_assign_kernel(const float4* __restrict__ x,
                                                                      const uint32_t* __restrict__ part,
                                                                      uint64_t n_blocks, int mode, uint32_t v,
                                                                      const float* __restrict__ cb,
                                                                      const FitState* __restrict__ st,
                                                                      uint16_t* __restrict__ key) {
  const uint64_t n_t = pass_len(st, mode, v, n_blocks);
  const uint64_t t0 = (uint64_t)blockIdx.x * kAssignThreads;
  if (t0 >= n_t) return;  // (whole workgroups)
  __shared__ float4 cent[kFitK];
  const float4* src = reinterpret_cast<const float4*>(cb) + (uint64_t)v * kFitK;
  for (uint32_t i = threadIdx.x; i < kFitK; i += kAssignThreads) cent[i] = src[i];
  __syncthreads();
  const uint64_t t = t0 + threadIdx.x;
  if (t >= n_t) return;
  const uint32_t* list = part + (v ? st->nm[0] : 0);
  const uint64_t blk = mode == kAll ? (t >> 2) : list[t >> 2];
  float d;
  key[t] = (uint16_t)nearest_entry(cent, x[blk * 4 + (t & 3)], d);
}

// Per-chunk key counts (one wave a chunk of kSortChunk keys): counts[chunk][key]. The wave requests
// all of its keys first (one per lane and step), then counts them step by step.
template <uint32_t NK, int BITS>
__global__ void __launch_bounds__(64) sort_count_kernel(const uint16_t* __restrict__ key, uint64_t n_blocks,
                                                        int mode, uint32_t v, const FitState* __restrict__ st,
                                                        uint32_t* __restrict__ counts) {
  const uint64_t n = pass_len(st, mode, v, n_blocks);
  const uint64_t e0 = (uint64_t)blockIdx.x * kSortChunk;
  if (e0 >= n) return;
  __shared__ uint32_t cnt[NK];
  const uint32_t lane = threadIdx.x;
  uint32_t kk[kSortSteps];
#pragma unroll
  for (uint32_t q = 0; q < kSortSteps; ++q) {
    const uint64_t el = e0 + 64u * q + lane;
    kk[q] = el < n ? key[el] : 0u;
  }
  for (uint32_t k = lane; k < NK; k += 64) cnt[k] = 0;
  __syncthreads();
#pragma unroll
  for (uint32_t q = 0; q < kSortSteps; ++q) {
    const bool valid = e0 + 64u * q + lane < n;
    const uint64_t m = same_key_lanes<BITS>(kk[q], valid);
    if (valid && (uint32_t)__builtin_ctzll(m) == lane) cnt[kk[q]] += (uint32_t)__popcll(m);
    __syncthreads();
  }
  for (uint32_t k = lane; k < NK; k += 64) counts[(uint64_t)blockIdx.x * NK + k] = cnt[k];
}

// counts[chunk][key] -> offset of the chunk's first key-k element within key k's run; segbase[k]
// = start of key k's run, segbase[NK] = n. The partition also records the member counts.
template <uint32_t NK>
__global__ void __launch_bounds__(1024) sort_scan_kernel(uint64_t n_blocks, int mode, uint32_t v,
                                                         FitState* __restrict__ st, uint32_t* __restrict__ counts,
                                                         uint32_t* __restrict__ segbase) {
  const uint64_t n = pass_len(st, mode, v, n_blocks);
  if (n == 0) return;
  __shared__ uint32_t sc[1024];
  const uint32_t n_w = (uint32_t)((n + kSortChunk - 1) / kSortChunk);
  const uint32_t k = threadIdx.x;
  uint32_t tot = 0;
  if (k < NK) {
    for (uint32_t w0 = 0; w0 < n_w; w0 += 16) {
      uint32_t cv[16];
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) cv[q] = w0 + q < n_w ? counts[(uint64_t)(w0 + q) * NK + k] : 0u;
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q)
        if (w0 + q < n_w) {
          counts[(uint64_t)(w0 + q) * NK + k] = tot;
          tot += cv[q];
        }
    }
  }
  const uint32_t incl = block_scan_incl<1024>(tot, sc);
  if (k < NK) segbase[k] = incl - tot;
  if (k == 0) segbase[NK] = (uint32_t)n;
  if (mode == kPartition && k < 2) st->nm[k] = tot;
}

// Stable scatter: each chunk's wave walks its keys in order; an element's place is its key's
// run start + the chunk's offset + the earlier equal keys of the chunk. The Lloyd passes move
// the item quads (xs, requested four steps ahead), the partition the block ids (part).
template <uint32_t NK, int BITS>
__global__ void __launch_bounds__(64) sort_scatter_kernel(const uint16_t* __restrict__ key, uint64_t n_blocks,
                                                          int mode, uint32_t v, const FitState* __restrict__ st,
                                                          const uint32_t* __restrict__ counts,
                                                          const uint32_t* __restrict__ segbase,
                                                          const float4* __restrict__ x, float4* __restrict__ xs,
                                                          uint32_t* __restrict__ part) {
  const uint64_t n = pass_len(st, mode, v, n_blocks);
  const uint64_t e0 = (uint64_t)blockIdx.x * kSortChunk;
  if (e0 >= n) return;
  __shared__ uint32_t runp[NK];
  const uint32_t lane = threadIdx.x;
  const uint32_t* list = mode == kMember ? part + (v ? st->nm[0] : 0) : nullptr;
  uint32_t kk[kSortSteps];
#pragma unroll
  for (uint32_t q = 0; q < kSortSteps; ++q) {
    const uint64_t el = e0 + 64u * q + lane;
    kk[q] = el < n ? key[el] : 0u;
  }
  auto quad = [&](uint32_t q) -> float4 {
    const uint64_t el = e0 + 64u * q + lane;
    if (mode == kPartition || el >= n) return make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const uint64_t blk = mode == kAll ? (el >> 2) : list[el >> 2];
    return x[blk * 4 + (el & 3)];
  };
  constexpr uint32_t kAhead = 4;
  float4 ring[kAhead];
#pragma unroll
  for (uint32_t q = 0; q < kAhead; ++q) ring[q] = quad(q);
  for (uint32_t k = lane; k < NK; k += 64) runp[k] = segbase[k] + counts[(uint64_t)blockIdx.x * NK + k];
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (uint32_t q = 0; q < kSortSteps; ++q) {
    const uint64_t el = e0 + 64u * q + lane;
    const bool valid = el < n;
    const uint32_t k = kk[q];
    const float4 xq = ring[q % kAhead];
    if (q + kAhead < kSortSteps) ring[q % kAhead] = quad(q + kAhead);
    const uint64_t m = same_key_lanes<BITS>(k, valid);
    const uint32_t pos = valid ? runp[k] + (uint32_t)__popcll(m & below) : 0u;
    __syncthreads();
    if (valid) {
      if ((uint32_t)__builtin_ctzll(m) == lane) runp[k] += (uint32_t)__popcll(m);
      if (mode == kPartition)
        part[pos] = (uint32_t)el;
      else
        xs[pos] = xq;
    }
    __syncthreads();
  }
}

// New centroids of variant v (blockquant.cpp:235-241): one thread per (entry, dimension) adds the
// entry's run of that dimension in item order (the run's values requested 16 ahead of the adds),
// divides by the count and rounds to float; |new - old| goes to diff[4 entry + dimension].
constexpr uint32_t kSumAhead = 16;
__global__ void __launch_bounds__(256) lloyd_sum_kernel(const float4* __restrict__ xs, uint64_t n_blocks, int mode,
                                                        uint32_t v, const uint32_t* __restrict__ segbase,
                                                        float* __restrict__ cb, float* __restrict__ diff,
                                                        const FitState* __restrict__ st) {
  if (pass_len(st, mode, v, n_blocks) == 0) return;
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;  // entry i / 4, dimension i % 4
  const uint32_t c = i >> 2, p = i & 3u;
  const uint32_t j0 = segbase[c], j1 = segbase[c + 1], cnt = j1 - j0;
  const float* src = reinterpret_cast<const float*>(xs + j0) + p;
  double acc = 0.0;
  float cur[kSumAhead], nxt[kSumAhead];
#pragma unroll
  for (uint32_t q = 0; q < kSumAhead; ++q) cur[q] = q < cnt ? src[4u * q] : 0.0f;
  for (uint32_t b = 0; b < cnt; b += kSumAhead) {
#pragma unroll
    for (uint32_t q = 0; q < kSumAhead; ++q) nxt[q] = b + kSumAhead + q < cnt ? src[4u * (b + kSumAhead + q)] : 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < kSumAhead; ++q)
      if (b + q < cnt) acc = acc + (double)cur[q];
#pragma unroll
    for (uint32_t q = 0; q < kSumAhead; ++q) cur[q] = nxt[q];
  }
  float* cent = cb + ((uint64_t)v * kFitK + c) * 4 + p;
  float d = 0.0f;  // an empty entry adds +0 to the shift, which leaves it as it is
  if (cnt > 0) {
    const float nv = (float)(acc / (double)cnt);
    d = fabsf(nv - *cent);
    *cent = nv;
  }
  diff[i] = d;
}

// The shift of the pass against 1e-7 (blockquant.cpp:242): the 4096 |new - old| are summed in
// parallel; any order of n non-negative additions lands within n * 2^-53 of the exact sum, the
// reference's entry-order sum included, so the comparison is decided from the parallel sum unless
// it lies within twice that bound of 1e-7 (or is NaN): then one lane repeats the sum in entry order.
__global__ void __launch_bounds__(256) lloyd_shift_kernel(const float* __restrict__ diff, uint64_t n_blocks, int mode,
                                                          uint32_t v, FitState* __restrict__ st) {
  if (pass_len(st, mode, v, n_blocks) == 0) return;
  __shared__ float buf[kFitK * 4];
  __shared__ double red[4];
  double part = 0.0;
  for (uint32_t i = threadIdx.x; i < kFitK * 4; i += 256) {
    const float d = diff[i];
    buf[i] = d;
    part = part + (double)d;
  }
  const double S = block_sum<256>(part, red);  // (thread 0)
  __syncthreads();
  if (threadIdx.x == 0) {
    const double G = (double)(kFitK * 4 + 64) * 0x1p-53 * 2.0;
    int done;
    if (S * (1.0 + G) < 1e-7) {
      done = 1;
    } else if (S * (1.0 - G) >= 1e-7) {
      done = 0;
    } else {  // (and NaN)
      double shift = 0.0;
      for (uint32_t i = 0; i < kFitK * 4; ++i) shift = shift + (double)buf[i];
      done = shift < 1e-7;
    }
    if (done) st->lloyd_done = 1u;
    st->n_passes += 1;
  }
}

__global__ void lloyd_begin_kernel(FitState* st) { st->lloyd_done = 0u; }

// Variant 1 = variant 0 * (float)exp2(1/2) (the octave seeding under power-of-two block scales,
// blockquant.cpp:328-339).
__global__ void __launch_bounds__(256) octave_kernel(float* __restrict__ cb, float m) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < kFitK * 4) cb[kFitK * 4 + i] = cb[i] * m;
}

// ---- block-level EM (blockquant.cpp:341-379) ---------------------------------------------------

__global__ void em_begin_kernel(FitState* st) { st->em_active = st->em_stop ? 0u : 1u; }

// Each block's better variant: the summed nearest distances of its four quads in double, strict
// <, variant 0 first (blockquant.cpp:348-362).
__global__ void __launch_bounds__(kAssignThreads) em_choice_kernel(const float4* __restrict__ x, uint64_t n_blocks,
                                                                   const float* __restrict__ cb,
                                                                   const FitState* __restrict__ st,
                                                                   uint16_t* __restrict__ ckey) {
  if (!st->em_active) return;
  __shared__ float4 cent[2 * kFitK];
  const float4* src = reinterpret_cast<const float4*>(cb);
  for (uint32_t i = threadIdx.x; i < 2 * kFitK; i += kAssignThreads) cent[i] = src[i];
  __syncthreads();
  const uint64_t t = (uint64_t)blockIdx.x * kAssignThreads + threadIdx.x;
  const bool valid = t < 4 * n_blocks;
  float d0 = 0.0f, d1 = 0.0f;
  if (valid) {
    const float4 xi = x[t];
    nearest_entry(cent, xi, d0);
    nearest_entry(cent + kFitK, xi, d1);
  }
  // the block's four quads are lanes 4j .. 4j + 3 of this wave
  const int g = (int)(threadIdx.x & 63) & ~3;
  float q0[4], q1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q0[i] = __uint_as_float((uint32_t)__builtin_amdgcn_ds_bpermute((g + i) << 2, (int)__float_as_uint(d0)));
    q1[i] = __uint_as_float((uint32_t)__builtin_amdgcn_ds_bpermute((g + i) << 2, (int)__float_as_uint(d1)));
  }
  if (valid && (t & 3) == 0) {
    double e0 = 0.0, e1 = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) e0 = e0 + (double)q0[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) e1 = e1 + (double)q1[i];
    uint32_t bestv = 0;
    double bestE = DBL_MAX;
    if (e0 < bestE) { bestE = e0; bestv = 0; }
    if (e1 < bestE) { bestE = e1; bestv = 1; }
    ckey[t >> 2] = (uint16_t)bestv;
  }
}

// An empty variant v is reseeded from variant 0 with the dither gap * 0.25 (v + 1), + on the
// first dimension and - on the others (blockquant.cpp:300-319, 373-374); the gap, the RMS of the
// samples over sqrt(1024), is summed by one lane in sample order, once.
__global__ void __launch_bounds__(64) em_reseed_kernel(const float* __restrict__ samples, uint64_t n_samples,
                                                       uint32_t v, float* __restrict__ cb, FitState* __restrict__ st) {
  if (!st->em_active || st->nm[v] != 0) return;
  __shared__ float buf[kSeqBuf];
  __shared__ double s_gap;
  const uint32_t lane = threadIdx.x;
  if (!st->gap_ready) {
    double sd = 0.0;
    for (uint64_t b0 = 0; b0 < n_samples; b0 += kSeqBuf) {
      for (uint32_t j = lane; j < kSeqBuf; j += 64) buf[j] = b0 + j < n_samples ? samples[b0 + j] : 0.0f;
      __syncthreads();
      if (lane == 0) {
        const uint32_t m = (uint32_t)(n_samples - b0 < kSeqBuf ? n_samples - b0 : kSeqBuf);
        for (uint32_t k = 0; k < m; ++k) sd = sd + (double)buf[k] * (double)buf[k];
      }
      __syncthreads();
    }
    if (lane == 0) {
      const double gap = sqrt(sd / (double)n_samples) / sqrt((double)kFitK);
      st->gap = gap;
      st->gap_ready = 1u;
      s_gap = gap;
    }
  } else if (lane == 0) {
    s_gap = st->gap;
  }
  __syncthreads();
  const double gap = s_gap, mult = 0.25 * (double)(v + 1);
  for (uint32_t i = lane; i < kFitK * 4; i += 64) {
    const uint32_t p = i & 3u;
    cb[(uint64_t)v * kFitK * 4 + i] = cb[i] + (float)(gap * mult * (p == 0 ? 1.0 : -1.0));
  }
}

__global__ void em_end_kernel(FitState* st) {
  if (!st->em_active) return;
  if (st->nm[0] == st->prev[0] && st->nm[1] == st->prev[1]) st->em_stop = 1u;
  st->prev[0] = st->nm[0];
  st->prev[1] = st->nm[1];
}

// ---- E4M3 projection and packing (blockquant.cpp:439-492) --------------------------------------

// The reference's table value of an E4M3 byte (src/quant/source_dtypes.cpp:14-32).
__device__ __forceinline__ float e4m3_value(uint32_t b) {
  if ((b & 0x7Fu) == 0x7Fu) return __uint_as_float(0x7FC00000u | ((b & 0x80u) << 24));
  return e4m3_to_f32(b);
}

// Nearest E4M3 byte over the 256 encodings, skipping NaN and every stored exponent outside 1..7,
// the first strict minimum of |value - x|.
__device__ __forceinline__ uint32_t e4m3_nearest_restricted(float x) {
  uint32_t best = 0;
  float bd = FLT_MAX;
  for (uint32_t i = 0; i < 256; ++i) {
    const uint32_t e = (i >> 3) & 15u;
    if ((i & 0x7Fu) == 0x7Fu || e == 0 || e > 7) continue;
    const float d = fabsf(e4m3_to_f32(i) - x);
    if (d < bd) {
      bd = d;
      best = i;
    }
  }
  return best;
}

__global__ void __launch_bounds__(256) project_kernel(float* __restrict__ cb, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) cb[i] = e4m3_to_f32(e4m3_nearest_restricted(cb[i]));
}

__global__ void __launch_bounds__(256) pack_kernel(const float* __restrict__ cb, uint32_t* __restrict__ packed) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= kVariants * kFitK) return;
  uint32_t w = 0;
#pragma unroll
  for (int p = 0; p < 4; ++p) w |= e4m3_nearest_restricted(cb[4 * i + p]) << (8 * p);
  packed[i] = w;
}

__global__ void __launch_bounds__(256) unpack_kernel(const uint32_t* __restrict__ packed, float* __restrict__ cb) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= kVariants * kFitK) return;
  const uint32_t w = packed[i];
#pragma unroll
  for (int p = 0; p < 4; ++p) cb[4 * i + p] = e4m3_value((w >> (8 * p)) & 0xFFu);
}

// ---- sample collection (blockquant.cpp:386-423) ------------------------------------------------

constexpr uint32_t kColThreads = 256;

__device__ __forceinline__ float block16_max(const float* blk) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock; ++i) m = fmaxf(m, fabsf(blk[i]));
  return m;
}

// Row j (= sampled row j * stride): the number of its 16-blocks that are kept (none when the
// row's max is 0; max ignores NaN, as std::max against a running 0 does).
__global__ void __launch_bounds__(kColThreads) collect_count_kernel(const float* __restrict__ w, uint64_t cols,
                                                                    uint64_t stride, uint32_t* __restrict__ rowcnt) {
  __shared__ float red[kColThreads / 64];
  __shared__ uint32_t redn[kColThreads / 64];
  const float* row = w + (uint64_t)blockIdx.x * stride * cols;
  float m = 0.0f;
  for (uint64_t c = threadIdx.x; c < cols; c += kColThreads) m = fmaxf(m, fabsf(row[c]));
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  const uint64_t nblk = cols / kBlock;
  uint32_t nz = 0;
  for (uint64_t b = threadIdx.x; b < nblk; b += kColThreads) nz += block16_max(row + b * kBlock) > 0.0f;
  for (int o = 32; o > 0; o >>= 1) nz += __shfl_xor(nz, o);
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = m;
    redn[threadIdx.x >> 6] = nz;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float rm = 0.0f;
    uint32_t n = 0;
    for (int i = 0; i < kColThreads / 64; ++i) {
      rm = fmaxf(rm, red[i]);
      n += redn[i];
    }
    rowcnt[blockIdx.x] = rm > 0.0f ? n : 0u;
  }
}

// Exclusive scan of the row counts (in blocks) and the total sample count.
__global__ void __launch_bounds__(1024) collect_scan_kernel(uint32_t* __restrict__ rowcnt, uint64_t n_rows,
                                                            uint64_t* __restrict__ n_out) {
  __shared__ uint64_t sc[1024];
  const uint64_t per = (n_rows + 1023) / 1024;
  const uint64_t r0 = threadIdx.x * per;
  uint64_t s = 0;
  for (uint64_t j = 0; j < per && r0 + j < n_rows; ++j) s += rowcnt[r0 + j];
  const uint64_t incl = block_scan_incl<1024>(s, sc);
  uint64_t run = incl - s;
  for (uint64_t j = 0; j < per && r0 + j < n_rows; ++j) {
    const uint32_t cv = rowcnt[r0 + j];
    rowcnt[r0 + j] = (uint32_t)run;
    run += cv;
  }
  if (threadIdx.x == 1023) *n_out = incl * kBlock;
}

// The kept blocks of row j, in column order, each divided by its max.
__global__ void __launch_bounds__(kColThreads) collect_write_kernel(const float* __restrict__ w, uint64_t cols,
                                                                    uint64_t stride, const uint32_t* __restrict__ rowoff,
                                                                    const uint32_t* __restrict__ rowkept,
                                                                    float* __restrict__ out, uint64_t cap) {
  __shared__ uint32_t sc[kColThreads];
  if (!rowkept[blockIdx.x]) return;  // (the row's max is 0)
  const float* row = w + (uint64_t)blockIdx.x * stride * cols;
  const uint64_t nblk = cols / kBlock;
  const uint64_t per = (nblk + kColThreads - 1) / kColThreads;
  const uint64_t b0 = threadIdx.x * per;
  uint32_t nz = 0;
  for (uint64_t j = 0; j < per && b0 + j < nblk; ++j) nz += block16_max(row + (b0 + j) * kBlock) > 0.0f;
  const uint32_t incl = block_scan_incl<kColThreads>(nz, sc);
  uint64_t pos = (uint64_t)rowoff[blockIdx.x] + (incl - nz);
  for (uint64_t j = 0; j < per && b0 + j < nblk; ++j) {
    const float* blk = row + (b0 + j) * kBlock;
    const float bm = block16_max(blk);
    if (!(bm > 0.0f)) continue;
    if ((pos + 1) * kBlock <= cap)
      for (int i = 0; i < kBlock; ++i) out[pos * kBlock + i] = blk[i] / bm;
    ++pos;
  }
}

// ---- host ----------------------------------------------------------------------------------------

uint64_t splitmix_next(uint64_t& z) {
  uint64_t x = (z += 0x9E3779B97F4A7C15ull);
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

struct FitWs {
  uint64_t st, d2, wgsum, key, ckey, counts, segbase, xs, part, diff, total;
};

FitWs fit_ws(uint64_t n_samples) {
  const uint64_t n_items = n_samples / 4, n_blocks = n_items / 4;
  const uint64_t n_kpp = (n_items + kKppChunk - 1) / kKppChunk;
  const uint64_t n_sort = (4 * n_blocks + kSortChunk - 1) / kSortChunk;
  FitWs w{};
  uint64_t o = 0;
  w.st = o; o += a256(sizeof(FitState));
  w.d2 = o; o += a256(n_items * 8);
  w.wgsum = o; o += a256(n_kpp * 8 + 8);
  w.key = o; o += a256(4 * n_blocks * 2 + 2);
  w.ckey = o; o += a256(n_blocks * 2 + 2);
  w.counts = o; o += a256((n_sort + 1) * kFitK * 4);
  w.segbase = o; o += a256((kFitK + 1) * 4);
  w.xs = o; o += a256(4 * n_blocks * 16 + 16);
  w.part = o; o += a256(n_blocks * 4 + 4);
  w.diff = o; o += a256(kFitK * 4 * 4);
  w.total = o;
  return w;
}

int fit_pass(int mode, uint32_t v, const float4* x, uint64_t n_blocks, float* cb, uint8_t* ws, const FitWs& L,
             hipStream_t s) {
  FitState* st = reinterpret_cast<FitState*>(ws + L.st);
  uint16_t* key = reinterpret_cast<uint16_t*>(ws + L.key);
  uint32_t* counts = reinterpret_cast<uint32_t*>(ws + L.counts);
  uint32_t* segbase = reinterpret_cast<uint32_t*>(ws + L.segbase);
  float4* xs = reinterpret_cast<float4*>(ws + L.xs);
  uint32_t* part = reinterpret_cast<uint32_t*>(ws + L.part);
  const uint64_t n_t = 4 * n_blocks;
  const uint32_t g_assign = (uint32_t)((n_t + kAssignThreads - 1) / kAssignThreads);
  const uint32_t g_sort = (uint32_t)((n_t + kSortChunk - 1) / kSortChunk);
  hipLaunchKernelGGL(lloyd_assign_kernel, dim3(g_assign), dim3(kAssignThreads), 0, s, x, part, n_blocks, mode, v,
                     cb, st, key);
  hipLaunchKernelGGL((sort_count_kernel<kFitK, 10>), dim3(g_sort), dim3(64), 0, s, key, n_blocks, mode, v, st,
                     counts);
  hipLaunchKernelGGL((sort_scan_kernel<kFitK>), dim3(1), dim3(1024), 0, s, n_blocks, mode, v, st, counts, segbase);
  hipLaunchKernelGGL((sort_scatter_kernel<kFitK, 10>), dim3(g_sort), dim3(64), 0, s, key, n_blocks, mode, v, st,
                     counts, segbase, x, xs, part);
  float* diff = reinterpret_cast<float*>(ws + L.diff);
  hipLaunchKernelGGL(lloyd_sum_kernel, dim3(kFitK * 4 / 256), dim3(256), 0, s, xs, n_blocks, mode, v, segbase, cb,
                     diff, st);
  hipLaunchKernelGGL(lloyd_shift_kernel, dim3(1), dim3(256), 0, s, diff, n_blocks, mode, v, st);
  return check_launch("fit: Lloyd pass");
}

}  // namespace
}  // namespace affx

using namespace affx;

extern "C" {

uint64_t affx_collect_samples_bound(uint64_t rows, uint64_t cols, uint64_t max_samples) {
  if (rows == 0 || cols == 0) return 0;
  const uint64_t total = rows * cols;
  const uint64_t budget = max_samples ? max_samples : 1;
  const uint64_t stride = total / budget > 1 ? total / budget : 1;
  const uint64_t n_rows = (rows + stride - 1) / stride;
  return n_rows * (cols / kBlock) * kBlock;
}

size_t affx_collect_samples_workspace_size(uint64_t rows, uint64_t cols, uint64_t max_samples) {
  if (rows == 0 || cols == 0) return 256;
  const uint64_t total = rows * cols;
  const uint64_t budget = max_samples ? max_samples : 1;
  const uint64_t stride = total / budget > 1 ? total / budget : 1;
  const uint64_t n_rows = (rows + stride - 1) / stride;
  return (size_t)a256(2 * n_rows * 4 + 8);
}

int affx_collect_samples(const float* w, uint64_t rows, uint64_t cols, uint64_t max_samples, float* out,
                         uint64_t cap, uint64_t* n_out, void* ws, size_t ws_bytes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!w || !out || !n_out || !ws || rows == 0 || cols == 0)
    return set_error(AFFX_ERR_ARG, "collect_samples: null pointer or empty matrix");
  const uint64_t total = rows * cols;
  const uint64_t budget = max_samples ? max_samples : 1;
  const uint64_t stride = total / budget > 1 ? total / budget : 1;
  const uint64_t n_rows = (rows + stride - 1) / stride;
  if (n_rows > 0x7FFFFFFFull || affx_collect_samples_bound(rows, cols, max_samples) / kBlock > 0xFFFFFFFFull)
    return set_error(AFFX_ERR_ARG, "collect_samples: %llu sampled rows is too many", (unsigned long long)n_rows);
  if (ws_bytes < affx_collect_samples_workspace_size(rows, cols, max_samples))
    return set_error(AFFX_ERR_ARG, "collect_samples: workspace of %zu bytes is too small", ws_bytes);
  uint32_t* rowcnt = static_cast<uint32_t*>(ws);
  uint32_t* rowkept = rowcnt + n_rows;
  hipLaunchKernelGGL(collect_count_kernel, dim3((uint32_t)n_rows), dim3(kColThreads), 0, stream, w, cols, stride,
                     rowcnt);
  if (int rc = check_launch("collect_count_kernel")) return rc;
  if (int rc = check_hip(hipMemcpyAsync(rowkept, rowcnt, n_rows * 4, hipMemcpyDeviceToDevice, stream),
                         "collect_samples: copy"))
    return rc;
  hipLaunchKernelGGL(collect_scan_kernel, dim3(1), dim3(1024), 0, stream, rowcnt, n_rows, n_out);
  if (int rc = check_launch("collect_scan_kernel")) return rc;
  hipLaunchKernelGGL(collect_write_kernel, dim3((uint32_t)n_rows), dim3(kColThreads), 0, stream, w, cols, stride,
                     rowcnt, rowkept, out, cap);
  return check_launch("collect_write_kernel");
}

size_t affx_fit_codebook_workspace_size(uint64_t n_samples) { return (size_t)fit_ws(n_samples).total; }

int affx_fit_codebook(const float* samples, uint64_t n_samples, const float* weights, uint32_t iters, uint64_t seed,
                      uint32_t flags, float* cb, void* ws, size_t ws_bytes, void* stream) {
  if (weights) return set_error(AFFX_DECLINED, "fit_codebook: importance weights are not supported");
  if (!cb || !ws || (n_samples >= 4 && !samples))
    return set_error(AFFX_ERR_ARG, "fit_codebook: null pointer");
  if ((reinterpret_cast<uintptr_t>(samples) & 15u) || (reinterpret_cast<uintptr_t>(cb) & 15u) ||
      (reinterpret_cast<uintptr_t>(ws) & 255u))
    return set_error(AFFX_ERR_ARG, "fit_codebook: samples and cb must be 16-byte, ws 256-byte aligned");
  const uint64_t n_items = n_samples / 4, n_blocks = n_items / 4;
  if (n_items >= (1ull << 32) / 2)
    return set_error(AFFX_ERR_ARG, "fit_codebook: %llu samples is too many", (unsigned long long)n_samples);
  const FitWs L = fit_ws(n_samples);
  if (ws_bytes < L.total) return set_error(AFFX_ERR_ARG, "fit_codebook: workspace of %zu bytes is too small", ws_bytes);
  uint8_t* wsb = static_cast<uint8_t*>(ws);
  FitState* st = reinterpret_cast<FitState*>(wsb + L.st);
  double* d2 = reinterpret_cast<double*>(wsb + L.d2);
  double* wgsum = reinterpret_cast<double*>(wsb + L.wgsum);
  uint16_t* ckey = reinterpret_cast<uint16_t*>(wsb + L.ckey);
  uint32_t* counts = reinterpret_cast<uint32_t*>(wsb + L.counts);
  uint32_t* segbase = reinterpret_cast<uint32_t*>(wsb + L.segbase);
  uint32_t* part = reinterpret_cast<uint32_t*>(wsb + L.part);
  const float4* x = reinterpret_cast<const float4*>(samples);
  hipStream_t s = static_cast<hipStream_t>(stream);

  hipLaunchKernelGGL(fit_init_kernel, dim3(1), dim3(256), 0, s, samples, n_items, cb, st);
  if (int rc = check_launch("fit_init_kernel")) return rc;
  if (n_items == 0) return AFFX_OK;

  // k-means++: the draws of the splitmix stream are host arithmetic, as in the reference
  const uint32_t n_kpp = (uint32_t)((n_items + kKppChunk - 1) / kKppChunk);
  uint64_t z = seed;
  for (uint32_t c = 1; c < kFitK; ++c) {
    const double a = (double)(splitmix_next(z) % 1000000ull) / 1e6;
    hipLaunchKernelGGL(kpp_update_kernel, dim3(n_kpp), dim3(kKppThreads), 0, s, x, n_items, cb, c, c == 1 ? 1 : 0,
                       d2, wgsum);
    hipLaunchKernelGGL(kpp_pick_kernel, dim3(1), dim3(kPickThreads), 0, s, x, n_items, d2, wgsum, n_kpp, a, c,
                       (flags & AFFX_FIT_SEQUENTIAL_PICKS) ? 1 : 0, cb, st);
    hipLaunchKernelGGL(kpp_seq_kernel, dim3(1), dim3(64), 0, s, x, n_items, d2, a, c, cb, st);
    if (int rc = check_launch("fit: k-means++ draw")) return rc;
  }
  if (n_blocks == 0) return AFFX_OK;

  // Lloyd over every block, variant 0
  hipLaunchKernelGGL(lloyd_begin_kernel, dim3(1), dim3(1), 0, s, st);
  for (uint32_t it = 0; it < iters; ++it)
    if (int rc = fit_pass(kAll, 0, x, n_blocks, cb, wsb, L, s)) return rc;

  // variant 1 an octave step above variant 0
  hipLaunchKernelGGL(octave_kernel, dim3(kFitK * 4 / 256), dim3(256), 0, s, cb, (float)std::exp2(1.0 / 2.0));

  // block-level EM
  const uint32_t g_choice = (uint32_t)((4 * n_blocks + kAssignThreads - 1) / kAssignThreads);
  const uint32_t g_part = (uint32_t)((n_blocks + kSortChunk - 1) / kSortChunk);
  for (uint32_t em = 0; em < kEmRounds; ++em) {
    hipLaunchKernelGGL(em_begin_kernel, dim3(1), dim3(1), 0, s, st);
    hipLaunchKernelGGL(em_choice_kernel, dim3(g_choice), dim3(kAssignThreads), 0, s, x, n_blocks, cb, st, ckey);
    hipLaunchKernelGGL((sort_count_kernel<2, 1>), dim3(g_part), dim3(64), 0, s, ckey, n_blocks, kPartition, 0u, st,
                       counts);
    hipLaunchKernelGGL((sort_scan_kernel<2>), dim3(1), dim3(1024), 0, s, n_blocks, kPartition, 0u, st, counts,
                       segbase);
    hipLaunchKernelGGL((sort_scatter_kernel<2, 1>), dim3(g_part), dim3(64), 0, s, ckey, n_blocks, kPartition, 0u,
                       st, counts, segbase, x, static_cast<float4*>(nullptr), part);
    if (int rc = check_launch("fit: EM partition")) return rc;
    for (uint32_t v = 0; v < kVariants; ++v) {
      hipLaunchKernelGGL(em_reseed_kernel, dim3(1), dim3(64), 0, s, samples, n_samples, v, cb, st);
      hipLaunchKernelGGL(lloyd_begin_kernel, dim3(1), dim3(1), 0, s, st);
      for (uint32_t it = 0; it < kEmIters; ++it)
        if (int rc = fit_pass(kMember, v, x, n_blocks, cb, wsb, L, s)) return rc;
    }
    hipLaunchKernelGGL(em_end_kernel, dim3(1), dim3(1), 0, s, st);
    if (int rc = check_launch("fit: EM round")) return rc;
  }
  return AFFX_OK;
}

int affx_fit_codebook_stats(const void* ws, uint64_t* seq_picks, uint64_t* passes, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!ws || !seq_picks || !passes) return set_error(AFFX_ERR_ARG, "fit_codebook_stats: null pointer");
  FitState h{};
  if (int rc = check_hip(hipMemcpyAsync(&h, ws, sizeof(h), hipMemcpyDeviceToHost, stream), "fit_codebook_stats"))
    return rc;
  if (int rc = check_hip(hipStreamSynchronize(stream), "fit_codebook_stats")) return rc;
  *seq_picks = h.n_seq_picks;
  *passes = h.n_passes;
  return AFFX_OK;
}

int affx_project_codebook(float* cb, uint64_t n, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!cb && n) return set_error(AFFX_ERR_ARG, "project_codebook: null pointer");
  if (n == 0) return AFFX_OK;
  hipLaunchKernelGGL(project_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream, cb, n);
  return check_launch("project_kernel");
}

int affx_pack_codebook(const float* cb, uint32_t* packed, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!cb || !packed) return set_error(AFFX_ERR_ARG, "pack_codebook: null pointer");
  hipLaunchKernelGGL(pack_kernel, dim3(kVariants * kFitK / 256), dim3(256), 0, stream, cb, packed);
  return check_launch("pack_kernel");
}

int affx_unpack_codebook(const uint32_t* packed, float* cb, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!cb || !packed) return set_error(AFFX_ERR_ARG, "unpack_codebook: null pointer");
  hipLaunchKernelGGL(unpack_kernel, dim3(kVariants * kFitK / 256), dim3(256), 0, stream, packed, cb);
  return check_launch("unpack_kernel");
}

}  // extern "C"
