// Single-matrix GEMV entries of the inner API: y += sum_i w[i] * (W_i . x) over up to 32
// quantised matrices of one shape, as the reference's expert_gemv_batch_hip and expert_gemv_hip
// (src/gpu/expert_kernel_hip.h:147-153, expert_kernel.hip:2687-2722, 2810-2819). They are what
// aff-gpucheck calls for its per-matrix GPU check and its GEMV bandwidth figure
// (tools/aff_gpucheck.cpp:278, 544-548).
//
// One workgroup per 16-row tile of y, 8 waves. The workgroup stages the codebook (rotated tables,
// KC interleaved copies) and the activation's three E4M3 terms (one exponent per 1024-column
// segment) in LDS, then each wave walks its (matrix, segment) units: a unit is one wave tile of
// the matrix (16 rows x 1024 columns, one 256-column run per lane), decoded step by step into
// MFMA A fragments and multiplied by the activation terms (v_mfma_scale_f32_16x16x128_f8f6f4,
// B columns 0-2 = the three terms). The next unit's weights are requested before the current
// one is computed. Per wave the units are summed in order, then the waves in order: every y
// element is one fixed-order sum (no atomics).
#include "affx_lut.h"

namespace affx {

constexpr int kGvMax = 32;       // matrices per launch (the reference's kMaxBatch)
constexpr int kGvW = 8;          // waves per workgroup
constexpr int kGvT = kGvW * 64;
constexpr int kGvKC = 4;         // codebook copies
constexpr int kGvChunk = 272;    // LDS bytes of one 256-column chunk of a term row (padded)
constexpr uint32_t kGvMaxCols = 8192;

struct GemvArgs {
  const uint8_t* codes[kGvMax];
  const uint8_t* fields[kGvMax];
  const uint16_t* rs[kGvMax];
  const float* w;      // device [n], or null: wscalar for every matrix
  float wscalar;
  uint32_t n, rows, cols;
  const uint32_t* codebook;
  const float* x;
  float* y;
};

__host__ __device__ inline uint32_t gv_row_bytes(uint32_t cols) { return (cols / kSegCols) * kGvChunk + 64u; }

template <int KC>
__global__ void __launch_bounds__(kGvT) gemv_kernel(GemvArgs A) {
  AFFX_DYN_LDS(lds);
  __shared__ __align__(16) uint32_t lut_s[Lut<KC, true>::kDwords];
  const uint8_t* lut = reinterpret_cast<const uint8_t*>(lut_s);
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rt = blockIdx.x, nseg = A.cols / kTileCols, nunit = A.n * nseg;
  const uint32_t rowb = gv_row_bytes(A.cols);
  uint8_t* xq = lds;                                                      // [3][rowb]
  int32_t* sig = reinterpret_cast<int32_t*>(lds + 3u * rowb);             // [nseg]
  float* part = reinterpret_cast<float*>(lds + 3u * rowb + 64u);          // [kGvW][16]
  const uint32_t copy4 = ((lane >> 1) & (KC - 1)) * 4u;
  const uint32_t c = lane & 15, kg = lane >> 4;

  // the small loads first (codebook, then this wave's activation segment; loads complete in issue
  // order, so waiting for them does not wait for the weights requested after them)
  uint32_t cbv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) cbv[i] = A.codebook[tid + (uint32_t)i * kGvT];
  // wave wv splits segment wv (at most 8 segments: cols <= 8192); the loads are unconditional
  // (a wave without a segment rereads the last one), so no branch holds them up
  const uint32_t sx = wv < nseg ? wv : nseg - 1u;
  float4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const float4*>(A.x + sx * kTileCols + 4u * (lane + 64u * i));
  // a unit's packed weights and the row scales of this lane's four accumulator rows
  Unit ua, ub;
  uint2 ra, rb;
  auto load = [&](Unit& u, uint2& r, uint32_t unit) {
    const uint32_t ok = unit < nunit;
    const uint32_t m = ok ? unit / nseg : 0u, s = ok ? unit % nseg : 0u;
    load_unit_ordered(u, A.codes[m], A.fields[m], (uint64_t)rt * nseg + s, lane);
    r = *reinterpret_cast<const uint2*>(A.rs[m] + rt * 16u + 4u * (lane >> 4));
  };
  load(ua, ra, wv);

  // activation terms: the segment's largest magnitude fixes its exponent (times 2^sigma in
  // [128, 256)), then three E4M3 terms per element
  if (wv < nseg) {
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const int sigma = mx > 0.f ? 7 - ilogbf(mx) : 0;
    if (lane == 0) sig[sx] = sigma;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t q0, q1, q2;
      split3x4(ldexpf(v[i].x, sigma), ldexpf(v[i].y, sigma), ldexpf(v[i].z, sigma), ldexpf(v[i].w, sigma), q0, q1, q2);
      const uint32_t col = (sx * 4u + (uint32_t)i) * kGvChunk + 4u * lane;
      *reinterpret_cast<uint32_t*>(xq + col) = q0;
      *reinterpret_cast<uint32_t*>(xq + rowb + col) = q1;
      *reinterpret_cast<uint32_t*>(xq + 2u * rowb + col) = q2;
    }
  }
  build_lut<KC, kGvT, 4, true>(lut_s, cbv, tid);
  __syncthreads();

  // lanes of columns 0-2 read term c of their K group; the others multiply zeros
  const bool used = c < 3u;
  float yacc[4] = {0.f, 0.f, 0.f, 0.f};
  uint32_t u = wv;
  for (; u < nunit; u += 2u * kGvW) {
    // two units per pass, so that each prefetch lands in the other register set
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t cur = u + (uint32_t)h * kGvW;
      if (cur >= nunit) break;
      Unit& U = h == 0 ? ua : ub;
      const uint2 rsv = h == 0 ? ra : rb;
      if (h == 0) load(ub, rb, cur + kGvW);  // the next unit (an absent one reloads unit 0)
      else load(ua, ra, cur + kGvW);
      const uint32_t m = cur / nseg, s = cur % nseg;
      const uint8_t* bsrc = xq + (used ? c : 0u) * rowb + (s * 4u + kg) * kGvChunk;
      v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
      uint32_t raw[8], bv[2];
      pin_step(U, 0);
      lut_lookup_step<KC, true>(U, lut, nullptr, copy4, 0, raw, bv);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        uint32_t nraw[8], nbv[2];
        if (st < 7) {
          AFFX_PIN(acc);
          pin_step(U, st + 1);
          lut_lookup_step<KC, true>(U, lut, nullptr, copy4, st + 1, nraw, nbv);
        }
        v8i b = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        if (used) {
          const u32x4 lo = *reinterpret_cast<const u32x4*>(bsrc + 32 * st);
          const u32x4 hi = *reinterpret_cast<const u32x4*>(bsrc + 32 * st + 16);
          b = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
        acc = mfma(lut_finish(raw, bv), b, acc);
        __builtin_amdgcn_sched_barrier(0);
        if (st < 7) {
#pragma unroll
          for (int i = 0; i < 8; ++i) raw[i] = nraw[i];
          bv[0] = nbv[0];
          bv[1] = nbv[1];
        }
      }
      // lane c = 0 of K group kg holds rows 4 kg + v: terms combined (columns 0, 1, 2), the
      // segment's exponent undone, row scale and matrix weight applied
      const float wm = A.w ? A.w[m] : A.wscalar;
      const float sc = ldexpf(wm, -sig[s]);
      const float rs[4] = {__uint_as_float(rsv.x << 16), __uint_as_float(rsv.x & 0xFFFF0000u),
                           __uint_as_float(rsv.y << 16), __uint_as_float(rsv.y & 0xFFFF0000u)};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float d = acc[v];
        const float val = d + row_shl<1>(d) * 0.0625f + row_shl<2>(d) * 0.00390625f;
        if (c == 0u) yacc[v] += val * rs[v] * sc;
      }
    }
  }
  if (c == 0u) {
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wv * 16u + 4u * kg + v] = yacc[v];
  }
  __syncthreads();
  if (tid < 16u) {
    float sum = 0.f;
    for (int q = 0; q < kGvW; ++q) sum += part[q * 16 + tid];
    A.y[rt * 16u + tid] += sum;
  }
}

}  // namespace affx

using namespace affx;

namespace {

int gemv_launch(const affx_matrix* mats, const float* weights, float wscalar, uint32_t n, const void* codebook,
                const float* x, float* y, hipStream_t st) {
  if (!mats || !codebook || !x || !y) return set_error(AFFX_ERR_ARG, "expert_gemv: null pointer");
  if (n == 0) return AFFX_OK;
  const uint32_t rows = mats[0].rows, cols = mats[0].cols;
  if (rows == 0 || rows % kTileRows || cols == 0 || cols % kTileCols || cols > kGvMaxCols)
    return set_error(AFFX_DECLINED, "expert_gemv: needs rows %% 16 == 0 and cols a multiple of 1024 up to %u "
                     "(got %u x %u)", kGvMaxCols, rows, cols);
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0)
    return set_error(AFFX_ERR_ARG, "expert_gemv: x must be 16-byte aligned");
  for (uint32_t i = 0; i < n; ++i)
    if (mats[i].rows != rows || mats[i].cols != cols || !mats[i].codes || !mats[i].fields || !mats[i].rscales)
      return set_error(AFFX_ERR_ARG, "expert_gemv: matrix %u is %ux%u (expected %ux%u) or has a null plane", i,
                       mats[i].rows, mats[i].cols, rows, cols);
  const uint32_t lds = 3u * gv_row_bytes(cols) + 64u + kGvW * 16u * 4u;
  int rc = check_hip(hipFuncSetAttribute((const void*)gemv_kernel<kGvKC>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)lds),
                     "hipFuncSetAttribute(gemv)");
  if (rc) return rc;
  // matrices in launches of at most 32, each accumulating into y after the one before
  for (uint32_t off = 0; off < n; off += kGvMax) {
    GemvArgs A{};
    A.n = n - off < (uint32_t)kGvMax ? n - off : (uint32_t)kGvMax;
    for (uint32_t i = 0; i < A.n; ++i) {
      A.codes[i] = (const uint8_t*)mats[off + i].codes;
      A.fields[i] = (const uint8_t*)mats[off + i].fields;
      A.rs[i] = (const uint16_t*)mats[off + i].rscales;
    }
    A.w = weights ? weights + off : nullptr;
    A.wscalar = wscalar;
    A.rows = rows;
    A.cols = cols;
    A.codebook = (const uint32_t*)codebook;
    A.x = x;
    A.y = y;
    hipLaunchKernelGGL(gemv_kernel<kGvKC>, dim3(rows / kTileRows), dim3(kGvT), lds, st, A);
    if ((rc = check_launch("gemv_kernel"))) return rc;
  }
  return AFFX_OK;
}

}  // namespace

extern "C" {

int affx_expert_gemv_batch(const affx_matrix* mats, const float* weights, uint32_t n_mats, const void* codebook,
                           const float* x, float* y, void* stream) {
  if (!weights && n_mats) return set_error(AFFX_ERR_ARG, "expert_gemv_batch: null weights");
  return gemv_launch(mats, weights, 0.f, n_mats, codebook, x, y, (hipStream_t)stream);
}

int affx_expert_gemv(const affx_matrix* m, const void* codebook, const float* x, float w, float* y,
                     void* stream) {
  const int rc = gemv_launch(m, nullptr, w, 1, codebook, x, y, (hipStream_t)stream);
  if (rc) return rc;
  // the reference's entry returns with the result in y (it synchronises the stream)
  return check_hip(hipStreamSynchronize((hipStream_t)stream), "expert_gemv sync");
}

}  // extern "C"
