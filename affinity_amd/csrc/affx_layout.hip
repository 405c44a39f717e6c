// Library plumbing, container geometry, the container <-> device layout permutation, the
// bit-exact dequantisation kernel and the fp8 MFMA self-test.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "affx_common.h"

namespace affx {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return AFFX_OK;
  return set_error(AFFX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

// ------------------------------------------------------------------------------------------------
// Geometry. The plane sizes follow the q2p875q4 row of kQuantTable (256-weight super-blocks of
// 80 B codes + 12 B fields, 2 B per row; src/format/aff_format.h:117-121) and the placement of
// compute_expert_layout: code planes, then field planes, then row scales, each 256 B aligned,
// stride 4 KiB aligned (src/format/aff_format.cpp:45-91).
// ------------------------------------------------------------------------------------------------
static uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

static uint64_t layout(uint64_t hidden, uint64_t inter, uint64_t* off, uint64_t* size) {
  const uint64_t rows[3] = {inter, inter, hidden}, cols[3] = {hidden, hidden, inter};
  uint64_t sz[9];
  for (int m = 0; m < 3; ++m) {
    const uint64_t sb = (rows[m] * cols[m] + 255) / 256;
    sz[3 * m + 0] = sb * 80;
    sz[3 * m + 1] = sb * 12;
    sz[3 * m + 2] = rows[m] * 2;
  }
  static const int order[9] = {0, 3, 6, 1, 4, 7, 2, 5, 8};
  uint64_t o = 0;
  for (int i = 0; i < 9; ++i) {
    const int p = order[i];
    if (off) off[p] = o;
    if (size) size[p] = sz[p];
    o = align_up(o + sz[p], 256);
  }
  return align_up(o, 4096);
}

static bool shape_ok(uint64_t hidden, uint64_t inter) {
  return hidden > 0 && inter > 0 && hidden % kTileCols == 0 && inter % kTileCols == 0 &&
         hidden % kTileRows == 0 && inter % kTileRows == 0;
}

// ------------------------------------------------------------------------------------------------
// Permutation. For one matrix [rows x cols]: unit (r, u) <-> (tile rt*nst + u/4, lane
// (r%16) + 16*(u%4)). Codes: 5 x 16 B chunks per unit at tile*5120 + j*1024 + lane*16. Fields:
// 12 B per unit at tile*768 + lane*12.
// ------------------------------------------------------------------------------------------------
struct MatPlanes {
  uint64_t rows, cols, code_off, field_off;
};

static void mats_of(uint64_t hidden, uint64_t inter, MatPlanes m[3]) {
  uint64_t off[9];
  layout(hidden, inter, off, nullptr);
  const uint64_t rows[3] = {inter, inter, hidden}, cols[3] = {hidden, hidden, inter};
  for (int i = 0; i < 3; ++i) m[i] = {rows[i], cols[i], off[3 * i], off[3 * i + 1]};
}

__host__ __device__ inline void unit_dest(uint64_t r, uint64_t u, uint64_t cols, uint64_t* tile,
                                          uint32_t* lane) {
  const uint64_t nst = cols / kTileCols;
  *tile = (r / kTileRows) * nst + u / 4;
  *lane = (uint32_t)(r % kTileRows + kTileRows * (u % 4));
}

// One matrix's code and field planes, container (row-major) <-> device (wave-tile) layout.
static void permute_matrix_host(const uint8_t* sc, const uint8_t* sf, uint8_t* dc, uint8_t* df, uint64_t rows,
                                uint64_t cols, bool to_device) {
  const uint64_t nseg = cols / kSegCols, crow = code_row_bytes(cols), frow = field_row_bytes(cols);
  for (uint64_t r = 0; r < rows; ++r)
    for (uint64_t u = 0; u < nseg; ++u) {
      uint64_t tile;
      uint32_t lane;
      unit_dest(r, u, cols, &tile, &lane);
      const uint64_t c_row = r * crow + u * kUnitCodeBytes;
      const uint64_t f_row = r * frow + u * kUnitFieldBytes;
      const uint64_t f_dev = tile * kTileFieldBytes + lane * kUnitFieldBytes;
      for (int j = 0; j < 5; ++j) {
        const uint64_t c_dev = tile * kTileCodeBytes + j * 1024 + lane * 16;
        if (to_device) std::memcpy(dc + c_dev, sc + c_row + 16 * j, 16);
        else std::memcpy(dc + c_row + 16 * j, sc + c_dev, 16);
      }
      if (to_device) std::memcpy(df + f_dev, sf + f_row, kUnitFieldBytes);
      else std::memcpy(df + f_row, sf + f_dev, kUnitFieldBytes);
    }
}

static void permute_host(const uint8_t* src, uint8_t* dst, uint64_t hidden, uint64_t inter,
                         bool to_device) {
  MatPlanes mp[3];
  mats_of(hidden, inter, mp);
  const uint64_t stride = layout(hidden, inter, nullptr, nullptr);
  std::memcpy(dst, src, stride);  // row scales and padding are not permuted
  for (int m = 0; m < 3; ++m)
    permute_matrix_host(src + mp[m].code_off, src + mp[m].field_off, dst + mp[m].code_off,
                        dst + mp[m].field_off, mp[m].rows, mp[m].cols, to_device);
}

// One thread per 16-byte code chunk or 12-byte field run; grid over (expert, matrix, unit).
__global__ void permute_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                               uint64_t stride, MatPlanes m0, MatPlanes m1, MatPlanes m2,
                               uint64_t units_per_expert, uint64_t n_experts) {
  const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t per_unit = 6;  // 5 code chunks + 1 field run
  const uint64_t total = n_experts * units_per_expert * per_unit;
  if (gid >= total) return;
  const uint64_t e = gid / (units_per_expert * per_unit);
  uint64_t rem = gid % (units_per_expert * per_unit);
  const uint32_t part = (uint32_t)(rem % per_unit);
  uint64_t unit = rem / per_unit;
  const MatPlanes* mp;
  const uint64_t n0 = m0.rows * (m0.cols / kSegCols), n1 = m1.rows * (m1.cols / kSegCols);
  if (unit < n0) mp = &m0;
  else if (unit < n0 + n1) { mp = &m1; unit -= n0; }
  else { mp = &m2; unit -= n0 + n1; }
  const uint64_t nseg = mp->cols / kSegCols, r = unit / nseg, u = unit % nseg;
  uint64_t tile;
  uint32_t lane;
  unit_dest(r, u, mp->cols, &tile, &lane);
  const uint8_t* s = src + e * stride;
  uint8_t* d = dst + e * stride;
  if (part < 5) {
    const uint64_t so = mp->code_off + r * (mp->cols * 10 / 32) + u * kUnitCodeBytes + 16 * part;
    const uint64_t dofs = mp->code_off + tile * kTileCodeBytes + part * 1024 + lane * 16;
    // source runs are 16 B aligned only per 80 B unit start; copy as 4 dwords (4 B aligned)
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(s + so);
    uint4 v = make_uint4(sp[0], sp[1], sp[2], sp[3]);
    *reinterpret_cast<uint4*>(d + dofs) = v;
  } else {
    const uint64_t so = mp->field_off + r * (mp->cols * 6 / 128) + u * kUnitFieldBytes;
    const uint64_t dofs = mp->field_off + tile * kTileFieldBytes + lane * kUnitFieldBytes;
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(s + so);
    uint32_t* dp = reinterpret_cast<uint32_t*>(d + dofs);
    dp[0] = sp[0];
    dp[1] = sp[1];
    dp[2] = sp[2];
  }
}

// Row scales and alignment padding are copied verbatim.
__global__ void copy_tail_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                 uint64_t stride, uint64_t tail_off, uint64_t n_experts) {
  const uint64_t words = (stride - tail_off) / 4;
  const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= words * n_experts) return;
  const uint64_t e = gid / words, w = gid % words;
  reinterpret_cast<uint32_t*>(dst + e * stride + tail_off)[w] =
      reinterpret_cast<const uint32_t*>(src + e * stride + tail_off)[w];
}

// ------------------------------------------------------------------------------------------------
// Dequantisation: one wave per 16x1024 tile, one lane per unit (row r, 256 columns). The codebook
// dword is fetched, rotated (g&2), sign-flipped (g&1) and exponent-shifted (s) exactly as the
// GEMM kernels do, its four E4M3 bytes decoded (exact) and multiplied by the bf16 row scale:
// rs * (+-2^s * e) has at most 8+4 significant bits, so the f32 product is exact and equals the
// reference's (rs * 2^s * +-1) * e bit for bit. src/quant/blockquant.cpp:793-833.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ codes,
                                                      const uint8_t* __restrict__ fields,
                                                      const uint16_t* __restrict__ rscales,
                                                      const uint32_t* __restrict__ codebook,
                                                      uint32_t rows, uint32_t cols,
                                                      float* __restrict__ out) {
  const uint32_t nst = cols / kTileCols;
  const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) / 64, lane = threadIdx.x % 64;
  const uint32_t n_tiles = rows / kTileRows * nst;
  if (wave >= n_tiles) return;
  const uint32_t rt = wave / nst, st = wave % nst;
  const uint32_t r = rt * kTileRows + lane % 16, u = st * 4 + lane / 16;
  uint32_t c[20], f[3];
  const uint8_t* cp = codes + (uint64_t)wave * kTileCodeBytes + lane * 16;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const uint4 v = *reinterpret_cast<const uint4*>(cp + j * 1024);
    c[4 * j] = v.x; c[4 * j + 1] = v.y; c[4 * j + 2] = v.z; c[4 * j + 3] = v.w;
  }
  const uint32_t* fp = reinterpret_cast<const uint32_t*>(fields + (uint64_t)wave * kTileFieldBytes + lane * 12);
  f[0] = fp[0]; f[1] = fp[1]; f[2] = fp[2];
  const float rs = __uint_as_float((uint32_t)rscales[r] << 16);
  float* orow = out + (uint64_t)r * cols + (uint64_t)u * kSegCols;
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    const uint32_t fb = stream_bits<3>(f, 6 * b, 6);
    const uint32_t var = fb >> 5, rot = (fb >> 4) & 1u;
    const uint32_t x = block_xor(fb), a = block_add(fb);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t code = stream_bits<20>(c, 10 * (4 * b + i), 10);
      uint32_t d = codebook[var * kLut + code];
      if (rot) d = __builtin_amdgcn_alignbit(d, d, 16);
      d = (d ^ x) + a;
      float4 o;
      o.x = rs * e4m3_to_f32(d & 0xFFu);
      o.y = rs * e4m3_to_f32((d >> 8) & 0xFFu);
      o.z = rs * e4m3_to_f32((d >> 16) & 0xFFu);
      o.w = rs * e4m3_to_f32(d >> 24);
      *reinterpret_cast<float4*>(orow + 16 * b + 4 * i) = o;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// MFMA self-test: one fp8 x fp8 16x16x128 product with unit E8M0 scales (127 = 2^0).
// ------------------------------------------------------------------------------------------------
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

__global__ void mfma_selftest_kernel(const uint32_t* __restrict__ a, const uint32_t* __restrict__ b,
                                     float* __restrict__ d) {
  const int l = threadIdx.x;
  v8i va, vb;
#pragma unroll
  for (int i = 0; i < 8; ++i) { va[i] = (int)a[l * 8 + i]; vb[i] = (int)b[l * 8 + i]; }
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(va, vb, acc, 0, 0, 0, 127, 0, 127);
#pragma unroll
  for (int i = 0; i < 4; ++i) d[l * 4 + i] = acc[i];
}

}  // namespace affx

using namespace affx;

static int g_cus = 0;

extern "C" {

const char* affx_last_error(void) { return g_err; }
const char* affx_version(void) { return "affx 0.1 gfx950"; }

int affx_init(void) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  hipDeviceProp_t p;
  rc = check_hip(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
  if (rc) return rc;
  if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
    return set_error(AFFX_ERR_DEVICE, "device %d is %s, this library is built for gfx950", dev,
                     p.gcnArchName);
  g_cus = p.multiProcessorCount;
  return noalloc_init_device(dev);
}

uint64_t affx_expert_layout(uint64_t hidden, uint64_t inter, uint64_t off9[9], uint64_t size9[9]) {
  return layout(hidden, inter, off9, size9);
}

int affx_codebook_valid(const uint32_t* cb) {
  if (!cb) return 0;
  for (int i = 0; i < kVariants * kLut; ++i)
    for (int p = 0; p < 4; ++p) {
      const uint32_t e = (cb[i] >> (8 * p + 3)) & 15u;
      if (e < 1 || e > 7) return 0;
    }
  return 1;
}

int affx_expert_to_device_layout(const void* src, void* dst, uint64_t hidden, uint64_t inter) {
  if (!src || !dst || src == dst || !shape_ok(hidden, inter))
    return set_error(AFFX_ERR_ARG, "expert_to_device_layout: bad arguments");
  permute_host((const uint8_t*)src, (uint8_t*)dst, hidden, inter, true);
  return AFFX_OK;
}

int affx_expert_from_device_layout(const void* src, void* dst, uint64_t hidden, uint64_t inter) {
  if (!src || !dst || src == dst || !shape_ok(hidden, inter))
    return set_error(AFFX_ERR_ARG, "expert_from_device_layout: bad arguments");
  permute_host((const uint8_t*)src, (uint8_t*)dst, hidden, inter, false);
  return AFFX_OK;
}

int affx_matrix_to_device_layout(const void* src_codes, const void* src_fields, void* dst_codes,
                                 void* dst_fields, uint32_t rows, uint32_t cols) {
  if (!src_codes || !src_fields || !dst_codes || !dst_fields || src_codes == dst_codes ||
      src_fields == dst_fields || rows == 0 || cols == 0 || rows % kTileRows || cols % kTileCols)
    return set_error(AFFX_ERR_ARG, "matrix_to_device_layout: bad arguments (rows %% 16, cols %% 1024)");
  permute_matrix_host((const uint8_t*)src_codes, (const uint8_t*)src_fields, (uint8_t*)dst_codes,
                      (uint8_t*)dst_fields, rows, cols, true);
  return AFFX_OK;
}

int affx_permute_experts(const void* src, void* dst, uint64_t n, uint64_t hidden, uint64_t inter,
                         void* stream) {
  if (!src || !dst || src == dst || !shape_ok(hidden, inter))
    return set_error(AFFX_ERR_ARG, "permute_experts: bad arguments");
  if (n == 0) return AFFX_OK;
  MatPlanes mp[3];
  mats_of(hidden, inter, mp);
  uint64_t off[9];
  const uint64_t stride = layout(hidden, inter, off, nullptr);
  uint64_t units = 0;
  for (int m = 0; m < 3; ++m) units += mp[m].rows * (mp[m].cols / kSegCols);
  hipStream_t s = (hipStream_t)stream;
  const uint64_t threads = n * units * 6;
  const uint64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7FFFFFFFull) return set_error(AFFX_ERR_ARG, "permute_experts: too many experts per call");
  hipLaunchKernelGGL(permute_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, (const uint8_t*)src,
                     (uint8_t*)dst, stride, mp[0], mp[1], mp[2], units, n);
  int rc = check_launch("permute_kernel");
  if (rc) return rc;
  const uint64_t tail = off[2];  // gate row scales: the first byte after the last field plane
  const uint64_t tw = (stride - tail) / 4 * n;
  hipLaunchKernelGGL(copy_tail_kernel, dim3((uint32_t)((tw + 255) / 256)), dim3(256), 0, s,
                     (const uint8_t*)src, (uint8_t*)dst, stride, tail, n);
  return check_launch("copy_tail_kernel");
}

int affx_dequant_matrix(const affx_matrix* m, const void* codebook, float* out, void* stream) {
  if (!m || !codebook || !out || !m->codes || !m->fields || !m->rscales)
    return set_error(AFFX_ERR_ARG, "dequant_matrix: null pointer");
  if (m->rows == 0 || m->rows % kTileRows || m->cols == 0 || m->cols % kTileCols)
    return set_error(AFFX_ERR_ARG, "dequant_matrix: rows %% 16 and cols %% 1024 must be 0 (got %ux%u)",
                     m->rows, m->cols);
  const uint32_t tiles = m->rows / kTileRows * (m->cols / kTileCols);
  hipLaunchKernelGGL(dequant_kernel, dim3((tiles + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)m->codes, (const uint8_t*)m->fields,
                     (const uint16_t*)m->rscales, (const uint32_t*)codebook, m->rows, m->cols, out);
  return check_launch("dequant_kernel");
}

int affx_selftest_mfma_fp8(const void* a, const void* b, float* d, void* stream) {
  if (!a || !b || !d) return set_error(AFFX_ERR_ARG, "selftest: null pointer");
  hipLaunchKernelGGL(mfma_selftest_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const uint32_t*)a, (const uint32_t*)b, d);
  return check_launch("mfma_selftest_kernel");
}

}  // extern "C"
