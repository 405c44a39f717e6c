/*
 * CPU oracle for the 2.875-bpw quad-codebook expert path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the product
 * never calls it. See oracle.h for conventions. Citations are file:line in the reference tree.
 *
 * Float semantics follow the reference exactly (same operation order, float vs double exactly
 * where the reference has them, no contraction: built with -ffp-contract=off). Loops that the
 * reference runs sequentially are parallelised here only where each output element is computed
 * by one thread in the reference's own order (rows of a matrix; the nearest-code search of the
 * Lloyd/EM passes, whose accumulation stays sequential), so results are bit-identical at any
 * thread count.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 0;
void orc_set_threads(int n) { g_threads = n > 0 ? n : 0; }
int orc_get_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }
#define NT orc_get_threads()

/* ------------------------------------------------------------------------------------------ */
/* element codecs                                                                              */
/* ------------------------------------------------------------------------------------------ */

/* OCP E4M3 "fn": bias 7, subnormals at E=0, S.1111.111 is NaN, no infinities.
 * src/quant/source_dtypes.cpp:91-112 */
float orc_e4m3_to_float(uint8_t b) {
  const int sign = b >> 7, e = (b >> 3) & 15, m = b & 7;
  float f;
  if (e == 0) f = ldexpf((float)m / 8.0f, -6);
  else if (e == 15 && m == 7) f = NAN;
  else f = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return sign ? -f : f;
}

/* Round-to-nearest-even by the carry trick; NaN payloads are not special-cased (the reference
 * does not either). src/quant/source_dtypes.h:40-46 */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* src/quant/source_dtypes.h:33-38 */
float orc_bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float g_e4m3[256];
static int g_e4m3_ready = 0;
static const float* e4m3_table(void) {
  if (!g_e4m3_ready) {
#pragma omp critical(orc_e4m3)
    {
      if (!g_e4m3_ready) {
        for (int i = 0; i < 256; ++i) g_e4m3[i] = orc_e4m3_to_float((uint8_t)i);
        g_e4m3_ready = 1;
      }
    }
  }
  return g_e4m3;
}

/* ------------------------------------------------------------------------------------------ */
/* bit streams: LSB-first, value bit j at stream bit index*bits + j.                           */
/* src/quant/blockquant.cpp:44-67                                                              */
/* ------------------------------------------------------------------------------------------ */

void orc_pack_bits(uint8_t* dst, uint64_t index, uint32_t bits, uint32_t value) {
  uint64_t pos = index * bits;
  for (uint32_t j = 0; j < bits; ++j, ++pos) {
    const uint8_t bit = (uint8_t)(1u << (pos & 7));
    if ((value >> j) & 1u) dst[pos >> 3] |= bit;
    else dst[pos >> 3] &= (uint8_t)~bit;
  }
}

uint32_t orc_unpack_bits(const uint8_t* src, uint64_t index, uint32_t bits) {
  uint64_t pos = index * bits;
  uint32_t v = 0;
  for (uint32_t j = 0; j < bits; ++j, ++pos) v |= (uint32_t)((src[pos >> 3] >> (pos & 7)) & 1u) << j;
  return v;
}

/* ------------------------------------------------------------------------------------------ */
/* synthetic inputs                                                                            */
/* ------------------------------------------------------------------------------------------ */

/* splitmix64 (Steele, Lea, Flood 2014) as src/quant/blockquant.cpp:37-42 advances it: draw k
 * (0-based) of a stream seeded `seed` is mix(seed + (k+1)*gamma). Written in this counter form so
 * that any draw can be computed independently. */
uint64_t orc_splitmix_at(uint64_t seed, uint64_t k) {
  uint64_t x = seed + (k + 1) * 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* Box-Muller, cosine branch, two draws per normal, in double: the generator of
 * src/quant/blockquant.cpp:862-869. */
static double normal_at(uint64_t seed, uint64_t i) {
  const double u1 = (double)((orc_splitmix_at(seed, 2 * i) >> 11) + 1) * (1.0 / 9007199254740992.0);
  const double u2 = (double)((orc_splitmix_at(seed, 2 * i + 1) >> 11) + 1) * (1.0 / 9007199254740992.0);
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_gen_normal_f64(uint64_t seed, uint64_t n, double* out) {
#pragma omp parallel for num_threads(NT) schedule(static)
  for (uint64_t i = 0; i < n; ++i) out[i] = normal_at(seed, i);
}

/* value i = bf16_RNE((float)(scale * N_i)), returned as the float it stands for. */
void orc_gen_normal_bf16(uint64_t seed, uint64_t n, double scale, float* out) {
#pragma omp parallel for num_threads(NT) schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    const float f = (float)(scale * normal_at(seed, i));
    out[i] = orc_bf16_to_f32(orc_f32_to_bf16(f));
  }
}

/* ------------------------------------------------------------------------------------------ */
/* container geometry: src/format/aff_format.h:102-122 (q2p875q4 row: 256-weight super-block,  */
/* 80 B codes, 12 B fields, 2 B per row) and aff_format.cpp:16-35, 45-91 (plane order and      */
/* 256 B / 4 KiB alignment).                                                                    */
/* ------------------------------------------------------------------------------------------ */

static uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

uint64_t orc_expert_layout(uint64_t hidden, uint64_t inter, uint64_t* off9, uint64_t* size9) {
  const uint64_t rows[3] = {inter, inter, hidden}, cols[3] = {hidden, hidden, inter};
  uint64_t sz[9];
  for (int m = 0; m < 3; ++m) {
    const uint64_t n = rows[m] * cols[m], sb = (n + 255) / 256;
    sz[3 * m + 0] = sb * 80;
    sz[3 * m + 1] = sb * 12;
    sz[3 * m + 2] = rows[m] * 2;
  }
  /* placement order: all code planes, then all field planes, then all row scales */
  const int order[9] = {0, 3, 6, 1, 4, 7, 2, 5, 8};
  uint64_t off = 0;
  for (int i = 0; i < 9; ++i) {
    const int p = order[i];
    if (off9) off9[p] = off;
    if (size9) size9[p] = sz[p];
    off = align_up(off + sz[p], 256);
  }
  return align_up(off, 4096);
}

/* ------------------------------------------------------------------------------------------ */
/* nearest quad: float distance, dimensions summed in order, first strict minimum.             */
/* src/quant/blockquant.cpp:162-174 (wide_argmin over a [dim][code] plane)                     */
/* ------------------------------------------------------------------------------------------ */

typedef struct { float d[4][ORC_LUT]; } Planes; /* one variant, SoA */

static void make_planes(const float* cb, uint32_t var, Planes* p) {
  for (uint32_t c = 0; c < ORC_LUT; ++c)
    for (uint32_t d = 0; d < 4; ++d) p->d[d][c] = cb[((size_t)var * ORC_LUT + c) * 4 + d];
}

static uint32_t nearest(const Planes* p, const float* x, float* out_d) {
  float s[ORC_LUT];
  const float x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
  for (uint32_t c = 0; c < ORC_LUT; ++c) {
    const float a = p->d[0][c] - x0, b = p->d[1][c] - x1, e = p->d[2][c] - x2, f = p->d[3][c] - x3;
    float t = a * a;
    t = t + b * b;
    t = t + e * e;
    t = t + f * f;
    s[c] = t;
  }
  float m = FLT_MAX;
  for (uint32_t c = 0; c < ORC_LUT; ++c) m = s[c] < m ? s[c] : m;
  uint32_t best = 0;
  if (m < FLT_MAX) {
    for (uint32_t c = 0; c < ORC_LUT; ++c)
      if (s[c] == m) { best = c; break; }
  }
  if (out_d) *out_d = m;
  return best;
}

/* ------------------------------------------------------------------------------------------ */
/* codebook fitting                                                                            */
/* ------------------------------------------------------------------------------------------ */

/* Every stride-th row (stride = max(1, rows*cols/budget)); skip all-zero rows and blocks; emit
 * blk[i]/bmax for each 16-block. src/quant/blockquant.cpp:386-423 */
uint64_t orc_collect_samples(const float* w, uint64_t rows, uint64_t cols, uint64_t budget,
                             float* out, uint64_t cap) {
  const uint64_t nblk = cols / ORC_BLOCK, total = rows * cols;
  const uint64_t stride = total / (budget ? budget : 1) > 1 ? total / (budget ? budget : 1) : 1;
  uint64_t n = 0;
  for (uint64_t r = 0; r < rows; r += stride) {
    const float* row = w + r * cols;
    float rmax = 0;
    for (uint64_t c = 0; c < cols; ++c) { const float a = fabsf(row[c]); rmax = rmax < a ? a : rmax; }
    if (rmax <= 0) continue;
    for (uint64_t b = 0; b < nblk; ++b) {
      const float* blk = row + b * ORC_BLOCK;
      float bmax = 0;
      for (int i = 0; i < ORC_BLOCK; ++i) { const float a = fabsf(blk[i]); bmax = bmax < a ? a : bmax; }
      if (bmax <= 0) continue;
      for (int i = 0; i < ORC_BLOCK; ++i, ++n)
        if (out && n < cap) out[n] = blk[i] / bmax;
    }
  }
  return n;
}

/* k-means refit of one variant over a list of blocks: assignment by nearest(), accumulation in
 * double in block order, centroid = (float)(sum/count), stop when the summed |shift| < 1e-7.
 * src/quant/blockquant.cpp:203-244 */
static void refit(float* cb, uint32_t var, const float* samples, const uint32_t* blocks,
                  uint64_t nb, uint32_t iters, uint32_t* assign, Planes* pl) {
  double* acc = (double*)malloc(sizeof(double) * ORC_LUT * 4);
  double* cnt = (double*)malloc(sizeof(double) * ORC_LUT);
  float* cent = cb + (size_t)var * ORC_LUT * 4;
  for (uint32_t it = 0; it < iters; ++it) {
    memset(acc, 0, sizeof(double) * ORC_LUT * 4);
    memset(cnt, 0, sizeof(double) * ORC_LUT);
    make_planes(cb, var, pl);
#pragma omp parallel for num_threads(NT) schedule(static)
    for (uint64_t j = 0; j < nb; ++j) {
      const uint64_t base = (uint64_t)blocks[j] * 4;
      for (int i = 0; i < 4; ++i) assign[j * 4 + i] = nearest(pl, samples + (base + i) * 4, NULL);
    }
    for (uint64_t j = 0; j < nb; ++j) {
      const uint64_t base = (uint64_t)blocks[j] * 4;
      for (int i = 0; i < 4; ++i) {
        const float* x = samples + (base + i) * 4;
        const uint32_t c = assign[j * 4 + i];
        for (int p = 0; p < 4; ++p) acc[c * 4 + p] += (double)x[p] * 1.0;
        cnt[c] += 1.0;
      }
    }
    double shift = 0;
    for (uint32_t c = 0; c < ORC_LUT; ++c) {
      if (cnt[c] <= 0) continue;
      for (int p = 0; p < 4; ++p) {
        const float nv = (float)(acc[c * 4 + p] / cnt[c]);
        shift += fabsf(nv - cent[c * 4 + p]);
        cent[c * 4 + p] = nv;
      }
    }
    if (shift < 1e-7) break;
  }
  free(acc);
  free(cnt);
}

/* Joint fit of the 2 x 1024 quad codebook (src/quant/blockquant.cpp:252-384, pair 4, pow2):
 *  1. k-means++ seeding of variant 0 with d2 carried forward (272-294), splitmix from `seed`;
 *  2. `iters` Lloyd passes over all blocks (296-299);
 *  3. variant 1 = variant 0 * (float)exp2(1/2) (321-339, octave seeding under pow2 scales);
 *  4. up to 12 EM rounds: each block picks the variant with the smaller summed nearest distance
 *     (strict <, variant ascending), each non-empty variant gets 6 Lloyd passes on its blocks,
 *     an empty one is reseeded as variant0 +- gap*0.25*(v+1); stop when member counts repeat
 *     (341-379). */
void orc_fit_codebook(const float* samples, uint64_t n_samples, uint32_t iters, uint64_t seed,
                      float* cb) {
  const uint64_t n_items = n_samples / 4;
  memset(cb, 0, sizeof(float) * ORC_VARIANTS * ORC_LUT * 4);
  if (n_items == 0) return;

  /* 1. k-means++ */
  uint64_t z = seed;
  for (int p = 0; p < 4; ++p) cb[p] = samples[p];
  double* d2 = (double*)malloc(sizeof(double) * n_items);
  for (uint64_t i = 0; i < n_items; ++i) d2[i] = DBL_MAX;
  for (uint32_t c = 1; c < ORC_LUT; ++c) {
    const float* last = cb + (size_t)(c - 1) * 4;
#pragma omp parallel for num_threads(NT) schedule(static)
    for (uint64_t i = 0; i < n_items; ++i) {
      const float* x = samples + i * 4;
      double s = 0;
      for (int p = 0; p < 4; ++p) { const double d = (double)x[p] - (double)last[p]; s += d * d; }
      s = 1.0 * s;
      if (s < d2[i]) d2[i] = s;
    }
    double tot = 0;
    for (uint64_t i = 0; i < n_items; ++i) tot += d2[i];
    /* draw k of the stream is mix(seed + (k+1)*gamma): the reference's `splitmix(z)` with z
     * advanced in place */
    const uint64_t r = orc_splitmix_at(z, 0);
    z += 0x9E3779B97F4A7C15ull;
    const double target = (double)(r % 1000000) / 1e6 * tot;
    double cum = 0;
    uint64_t pick = n_items - 1;
    for (uint64_t i = 0; i < n_items; ++i) {
      cum += d2[i];
      if (cum >= target) { pick = i; break; }
    }
    for (int p = 0; p < 4; ++p) cb[(size_t)c * 4 + p] = samples[pick * 4 + p];
  }
  free(d2);

  const uint64_t n_blocks = n_items / 4;
  if (n_blocks == 0) return;
  uint32_t* all = (uint32_t*)malloc(sizeof(uint32_t) * n_blocks);
  uint32_t* assign = (uint32_t*)malloc(sizeof(uint32_t) * n_blocks * 4);
  Planes* pl = (Planes*)malloc(sizeof(Planes) * 2);
  for (uint64_t b = 0; b < n_blocks; ++b) all[b] = (uint32_t)b;

  /* 2. Lloyd on variant 0 */
  refit(cb, 0, samples, all, n_blocks, iters, assign, &pl[0]);

  /* 3. octave seeding of variant 1 */
  double sd = 0;
  for (uint64_t i = 0; i < n_samples; ++i) sd += (double)samples[i] * (double)samples[i];
  const double gap = sqrt(sd / (double)n_samples) / sqrt((double)ORC_LUT);
  const float mult = (float)exp2(1.0 / 2.0);
  for (uint32_t c = 0; c < ORC_LUT; ++c)
    for (int p = 0; p < 4; ++p) cb[((size_t)ORC_LUT + c) * 4 + p] = cb[(size_t)c * 4 + p] * mult;

  /* 4. block-level EM */
  uint32_t* members[2];
  members[0] = (uint32_t*)malloc(sizeof(uint32_t) * n_blocks);
  members[1] = (uint32_t*)malloc(sizeof(uint32_t) * n_blocks);
  uint8_t* choice = (uint8_t*)malloc(n_blocks);
  uint64_t prev[2] = {UINT64_MAX, UINT64_MAX};
  for (uint32_t em = 0; em < 12; ++em) {
    make_planes(cb, 0, &pl[0]);
    make_planes(cb, 1, &pl[1]);
#pragma omp parallel for num_threads(NT) schedule(static)
    for (uint64_t b = 0; b < n_blocks; ++b) {
      uint32_t bestv = 0;
      double bestE = DBL_MAX;
      for (uint32_t v = 0; v < 2; ++v) {
        double e = 0;
        for (int i = 0; i < 4; ++i) {
          float d;
          nearest(&pl[v], samples + (b * 4 + i) * 4, &d);
          e += (double)d * 1.0;
        }
        if (e < bestE) { bestE = e; bestv = v; }
      }
      choice[b] = (uint8_t)bestv;
    }
    uint64_t nm[2] = {0, 0};
    for (uint64_t b = 0; b < n_blocks; ++b) members[choice[b]][nm[choice[b]]++] = (uint32_t)b;
    for (uint32_t v = 0; v < 2; ++v) {
      if (nm[v] == 0) {
        const double m2 = 0.25 * (double)(v + 1);
        for (uint32_t c = 0; c < ORC_LUT; ++c)
          for (int p = 0; p < 4; ++p)
            cb[((size_t)v * ORC_LUT + c) * 4 + p] =
                cb[(size_t)c * 4 + p] + (float)(gap * m2 * (p == 0 ? 1.0 : -1.0));
      } else {
        refit(cb, v, samples, members[v], nm[v], 6, assign, &pl[v]);
      }
    }
    if (nm[0] == prev[0] && nm[1] == prev[1]) break;
    prev[0] = nm[0];
    prev[1] = nm[1];
  }
  free(members[0]);
  free(members[1]);
  free(choice);
  free(pl);
  free(assign);
  free(all);
}

/* Nearest E4M3 byte by exhaustive scan over the 256 encodings, skipping NaN and (pow2 block
 * scales) every stored exponent outside 1..7; ties keep the lowest byte.
 * src/quant/blockquant.cpp:439-461 */
uint8_t orc_e4m3_nearest(float x) {
  const float* t = e4m3_table();
  int best = 0;
  float bd = FLT_MAX;
  for (int i = 0; i < 256; ++i) {
    if ((i & 0x7f) == 0x7f) continue;
    const int e = (i >> 3) & 15;
    if (e == 0 || e > 7) continue;
    const float d = fabsf(t[i] - x);
    if (d < bd) { bd = d; best = i; }
  }
  return (uint8_t)best;
}

/* src/quant/blockquant.cpp:463-466 */
void orc_project_codebook(float* cb, uint64_t n) {
  const float* t = e4m3_table();
  for (uint64_t i = 0; i < n; ++i) cb[i] = t[orc_e4m3_nearest(cb[i])];
}

/* src/quant/blockquant.cpp:468-480 */
void orc_pack_codebook(const float* cb, uint32_t* packed) {
  for (uint32_t i = 0; i < ORC_VARIANTS * ORC_LUT; ++i) {
    uint32_t w = 0;
    for (int p = 0; p < 4; ++p) w |= (uint32_t)orc_e4m3_nearest(cb[(size_t)i * 4 + p]) << (8 * p);
    packed[i] = w;
  }
}

/* src/quant/blockquant.cpp:482-492 */
void orc_unpack_codebook(const uint32_t* packed, float* cb) {
  const float* t = e4m3_table();
  for (uint32_t i = 0; i < ORC_VARIANTS * ORC_LUT; ++i)
    for (int p = 0; p < 4; ++p) cb[(size_t)i * 4 + p] = t[(packed[i] >> (8 * p)) & 0xffu];
}

/* The load-time check that every codebook byte has stored exponent 1..7 (the condition under
 * which the block scale is an exponent add): src/gpu/static_placement.hip:938-951. */
int orc_codebook_exponents_ok(const uint32_t* packed) {
  for (uint32_t i = 0; i < ORC_VARIANTS * ORC_LUT; ++i)
    for (int p = 0; p < 4; ++p) {
      const uint32_t e = (packed[i] >> (8 * p + 3)) & 15u;
      if (e < 1 || e > 7) return 0;
    }
  return 1;
}

/* ------------------------------------------------------------------------------------------ */
/* quantise / dequantise                                                                       */
/* ------------------------------------------------------------------------------------------ */

/* One matrix, rows independent (src/quant/blockquant.cpp:586-791, quad format):
 *  rscale = bf16(ldexp(rmax, -7)) used at its stored value (648-665);
 *  per block: mid = first s in 0..7 minimising |2^s - bmax/rscale| (double), window
 *  [mid-1, mid+1] (686-705); search v -> s -> g, score = (double)(sum_quads float(min dist)*wt)
 *  * bs * bs with bs = rscale*2^s, targets blk[4i+(p+rh)%4] * (+-1/bs), first strict minimum
 *  (706-762); field = v<<5 | g<<3 | s (765-766); codes = nearest quad of blk[..]/(+-mag) with
 *  a division (768-786), all zero when mag <= 0. */
int orc_quantize_matrix(const float* w, uint64_t rows, uint64_t cols, const float* cb,
                        const float* col_importance, uint8_t* codes, uint8_t* fields,
                        uint16_t* rscales) {
  if (cols % ORC_BLOCK != 0 || cols == 0) return -1;
  const uint64_t nblk = cols / ORC_BLOCK, codes_row = cols / 4;
  Planes* pl = (Planes*)malloc(sizeof(Planes) * 2);
  make_planes(cb, 0, &pl[0]);
  make_planes(cb, 1, &pl[1]);
  /* the streams are byte-aligned per row (10*cols/4 and 6*cols/16 bits are multiples of 8
   * whenever cols % 64 == 0); clear them first so rows can be packed independently */
  memset(codes, 0, (rows * codes_row * 10 + 7) / 8);
  memset(fields, 0, (rows * nblk * 6 + 7) / 8);
  const int row_parallel = (cols % 64) == 0;
#pragma omp parallel for num_threads(row_parallel ? NT : 1) schedule(dynamic, 4)
  for (uint64_t r = 0; r < rows; ++r) {
    const float* row = w + r * cols;
    float rmax = 0;
    for (uint64_t c = 0; c < cols; ++c) { const float a = fabsf(row[c]); rmax = rmax < a ? a : rmax; }
    float rscale = rmax > 0 ? ldexpf(rmax, -ORC_BIAS) : 0.0f;
    const uint16_t h = orc_f32_to_bf16(rscale);
    rscales[r] = h;
    rscale = orc_bf16_to_f32(h);
    for (uint64_t b = 0; b < nblk; ++b) {
      const float* blk = row + b * ORC_BLOCK;
      float bmax = 0;
      for (int i = 0; i < ORC_BLOCK; ++i) { const float a = fabsf(blk[i]); bmax = bmax < a ? a : bmax; }
      uint32_t best_s = 0, best_v = 0, best_g = 0;
      double best_err = DBL_MAX;
      if (bmax > 0 && rscale > 0) {
        const double ideal = (double)bmax / (double)rscale;
        uint32_t mid = 0;
        double bd = DBL_MAX;
        for (uint32_t s = 0; s <= 7; ++s) {
          const double d = fabs((double)(float)(1u << s) - ideal);
          if (d < bd) { bd = d; mid = s; }
        }
        const int lo = (int)mid - 1 > 0 ? (int)mid - 1 : 0;
        const int hi = (int)mid + 1 < 7 ? (int)mid + 1 : 7;
        for (uint32_t v = 0; v < 2; ++v) {
          for (int s = lo; s <= hi; ++s) {
            const float bs = rscale * (float)(1u << s);
            if (bs <= 0) continue;
            const float inv = 1.0f / bs;
            for (uint32_t g = 0; g < 4; ++g) {
              const float sg = (g & 1u) ? -inv : inv;
              const uint32_t rh = (g & 2u) ? 2u : 0u;
              float acc = 0.0f;
              for (int i = 0; i < 4; ++i) {
                float t[4];
                for (uint32_t p = 0; p < 4; ++p) t[p] = blk[i * 4 + (p + rh) % 4] * sg;
                float wt = 1.0f;
                if (col_importance) {
                  const uint64_t c0 = b * ORC_BLOCK + (uint64_t)i * 4;
                  wt = 0.0f;
                  for (int p = 0; p < 4; ++p) wt += col_importance[c0 + p];
                  wt /= 4.0f;
                }
                float d;
                nearest(&pl[v], t, &d);
                acc += d * wt;
              }
              const double e = (double)acc * (double)bs * (double)bs;
              if (e < best_err) { best_err = e; best_s = (uint32_t)s; best_v = v; best_g = g; }
            }
          }
        }
      }
      orc_pack_bits(fields, r * nblk + b, 6, (best_v << 5) | (best_g << 3) | best_s);
      const float mag = rscale * (float)(1u << best_s);
      const float bs = (best_g & 1u) ? -mag : mag;
      const uint32_t rh = (best_g & 2u) ? 2u : 0u;
      const uint64_t code_base = r * codes_row + b * 4;
      if (mag <= 0) {
        for (int i = 0; i < 4; ++i) orc_pack_bits(codes, code_base + i, 10, 0);
        continue;
      }
      for (int i = 0; i < 4; ++i) {
        float t[4];
        for (uint32_t p = 0; p < 4; ++p) t[p] = blk[i * 4 + (p + rh) % 4] / bs;
        orc_pack_bits(codes, code_base + i, 10, nearest(&pl[best_v], t, NULL));
      }
    }
  }
  free(pl);
  return 0;
}

/* w = (rscale * 2^s * (+-1)) * e[v][code][(p+rh)%4] in float, v clamped to the last variant.
 * src/quant/blockquant.cpp:793-833 */
int orc_dequantize_matrix(const uint8_t* codes, const uint8_t* fields, const uint16_t* rscales,
                          uint64_t rows, uint64_t cols, const float* cb, float* out) {
  if (cols % ORC_BLOCK != 0) return -1;
  const uint64_t nblk = cols / ORC_BLOCK, codes_row = cols / 4;
#pragma omp parallel for num_threads(NT) schedule(static)
  for (uint64_t r = 0; r < rows; ++r) {
    const float rscale = orc_bf16_to_f32(rscales[r]);
    float* orow = out + r * cols;
    for (uint64_t b = 0; b < nblk; ++b) {
      const uint32_t f = orc_unpack_bits(fields, r * nblk + b, 6);
      const uint32_t s = f & 7u, g = (f >> 3) & 3u;
      const uint32_t v = (f >> 5) < 1u ? (f >> 5) : 1u;
      const float bs = rscale * (float)(1u << s) * ((g & 1u) ? -1.0f : 1.0f);
      const uint32_t rh = (g & 2u) ? 2u : 0u;
      for (int i = 0; i < 4; ++i) {
        const uint32_t c = orc_unpack_bits(codes, r * codes_row + b * 4 + i, 10);
        const float* e = cb + ((size_t)v * ORC_LUT + c) * 4;
        for (uint32_t p = 0; p < 4; ++p) orow[b * ORC_BLOCK + i * 4 + p] = bs * e[(p + rh) % 4];
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* CPU expert compute                                                                          */
/* ------------------------------------------------------------------------------------------ */

/* y[r] += w * (float)(sum_{b,i,p} (double)(bs*e[(p+rh)%4]) * (double)x[c]): the scalar
 * double-accumulating reference the quad format always takes
 * (src/engine/expert_kernel.cpp:64-101 for the sum, 126-139 for the tmp-then-scale step). */
void orc_expert_gemv(const uint8_t* codes, const uint8_t* fields, const uint16_t* rscales,
                     uint64_t rows, uint64_t cols, const float* cb, const float* x, float w,
                     float* y) {
  const uint64_t nblk = cols / ORC_BLOCK, codes_row = cols / 4;
#pragma omp parallel for num_threads(NT) schedule(static)
  for (uint64_t r = 0; r < rows; ++r) {
    const float rs = orc_bf16_to_f32(rscales[r]);
    double acc = 0.0;
    for (uint64_t b = 0; b < nblk; ++b) {
      const uint32_t f = orc_unpack_bits(fields, r * nblk + b, 6);
      const uint32_t g = (f >> 3) & 3u, var = f >> 5;
      const float bs = rs * (float)(1u << (f & 7u)) * ((g & 1u) ? -1.0f : 1.0f);
      const uint32_t rh = (g & 2u) ? 2u : 0u;
      const float* lut = cb + (size_t)(var < 2 ? var : 0) * ORC_LUT * 4;
      for (int i = 0; i < 4; ++i) {
        const uint32_t code = orc_unpack_bits(codes, r * codes_row + b * 4 + i, 10);
        const float* e = lut + (size_t)code * 4;
        const uint64_t c0 = b * ORC_BLOCK + (uint64_t)i * 4;
        for (uint32_t p = 0; p < 4; ++p) acc += (double)(bs * e[(p + rh) % 4]) * (double)x[c0 + p];
      }
    }
    const float tmp = 0.0f + (float)acc;
    y[r] += w * tmp;
  }
}

/* a = (g'/(1+exp(-g'))) * u' with g' = min(g, L), u' = clamp(u, -L, L) when L > 0, using the
 * comparison forms of std::min/std::max. src/engine/ops.cpp:47-60 */
void orc_swiglu(const float* gate, const float* up, uint64_t n, float limit, float* out) {
  for (uint64_t i = 0; i < n; ++i) {
    float g = gate[i], u = up[i];
    if (limit > 0.0f) {
      g = (limit < g) ? limit : g;
      const float lo = (-limit < u) ? u : -limit;
      u = (lo < limit) ? lo : limit;
    }
    out[i] = (g / (1.0f + expf(-g))) * u;
  }
}

/* One routed expert on one token: y += w * W_d . swiglu(W_g x, W_u x), the CPU composition of
 * src/engine/model.cpp:1187-1198. `expert` points at the expert's bytes in container layout. */
void orc_expert_ffn(const uint8_t* expert, uint64_t hidden, uint64_t inter, const float* cb,
                    const float* x, float w, float limit, float* y) {
  uint64_t off[9], size[9];
  orc_expert_layout(hidden, inter, off, size);
  float* g = (float*)calloc(inter, sizeof(float));
  float* u = (float*)calloc(inter, sizeof(float));
  float* a = (float*)calloc(inter, sizeof(float));
  orc_expert_gemv(expert + off[0], expert + off[1], (const uint16_t*)(expert + off[2]), inter,
                  hidden, cb, x, 1.0f, g);
  orc_expert_gemv(expert + off[3], expert + off[4], (const uint16_t*)(expert + off[5]), inter,
                  hidden, cb, x, 1.0f, u);
  orc_swiglu(g, u, inter, limit, a);
  orc_expert_gemv(expert + off[6], expert + off[7], (const uint16_t*)(expert + off[8]), hidden,
                  inter, cb, a, w, y);
  free(g);
  free(u);
  free(a);
}

/* ------------------------------------------------------------------------------------------ */
/* routing of the synthetic configs: softmax over the logits, top-k by logit (ties -> lower    */
/* id), weights renormalised over the k. The engine's own router (sqrtsoftplus + bias, x1.5,   */
/* src/engine/ops.cpp:62-92) is the caller's business; the configs fix this rule instead.      */
/* ------------------------------------------------------------------------------------------ */
void orc_route_softmax_topk(const float* logits, uint32_t n_expert, uint32_t k, uint32_t* sel,
                            float* w) {
  uint8_t* taken = (uint8_t*)calloc(n_expert, 1);
  float m = logits[0];
  for (uint32_t e = 1; e < n_expert; ++e) m = logits[e] > m ? logits[e] : m;
  double ex[64], sum = 0;
  for (uint32_t j = 0; j < k; ++j) {
    uint32_t best = UINT32_MAX;
    for (uint32_t e = 0; e < n_expert; ++e)
      if (!taken[e] && (best == UINT32_MAX || logits[e] > logits[best])) best = e;
    taken[best] = 1;
    sel[j] = best;
    ex[j] = exp((double)logits[best] - (double)m);
    sum += ex[j];
  }
  for (uint32_t j = 0; j < k; ++j) w[j] = (float)(ex[j] / sum);
  free(taken);
}

/* The engine's router (src/engine/ops.cpp:30-35 sqrtsoftplus, 62-92 route_topk): score =
 * sqrt(softplus(logit)) with the x > 20 guard, all in float (expf, log1pf, sqrtf: the float
 * overloads std::exp/std::log1p/std::sqrt call); selection value = score + bias; the k best by
 * selection value, ties to the lower id (std::partial_sort with that strict order picks exactly
 * these, in that order); weights from the scores only: sum in double, floored at the fp16 least
 * normal, weight = (float)(score * inv * routed_scaling) with inv = 1/sum when norm_topk_prob.
 * Returns the number of experts chosen (min(k, n_expert)). */
float orc_sqrtsoftplus(float x) {
  const float sp = (x > 20.0f) ? x : log1pf(expf(x));
  return sqrtf(sp);
}

uint32_t orc_route_topk(const float* logits, const float* bias, uint32_t n_expert, uint32_t k,
                        int norm_topk_prob, float routed_scaling, uint32_t* sel, float* w) {
  float* score = (float*)malloc(sizeof(float) * n_expert);
  float* key = (float*)malloc(sizeof(float) * n_expert);
  uint8_t* taken = (uint8_t*)calloc(n_expert, 1);
  for (uint32_t e = 0; e < n_expert; ++e) {
    score[e] = orc_sqrtsoftplus(logits[e]);
    key[e] = score[e] + (bias ? bias[e] : 0.0f);
  }
  const uint32_t kk = k < n_expert ? k : n_expert;
  for (uint32_t j = 0; j < kk; ++j) {
    uint32_t best = UINT32_MAX;
    for (uint32_t e = 0; e < n_expert; ++e) {
      if (taken[e]) continue;
      if (best == UINT32_MAX || key[e] > key[best]) best = e; /* equal keys keep the lower id */
    }
    taken[best] = 1;
    sel[j] = best;
  }
  double sum = 0.0;
  for (uint32_t j = 0; j < kk; ++j) sum += score[sel[j]];
  if (sum < 6.103515625e-5) sum = 6.103515625e-5;
  const double inv = norm_topk_prob ? 1.0 / sum : 1.0;
  for (uint32_t j = 0; j < kk; ++j) w[j] = (float)(score[sel[j]] * inv * routed_scaling);
  free(score);
  free(key);
  free(taken);
  return kk;
}

/* ------------------------------------------------------------------------------------------ */
/* the step after the routed experts                                                           */
/* ------------------------------------------------------------------------------------------ */

/* UE8M0: 2^(e - 127), 0xFF is NaN (src/quant/source_dtypes.cpp:41-50). */
float orc_e8m0_to_float(uint8_t e) { return e == 0xFF ? NAN : ldexpf(1.0f, (int)e - 127); }

/* FP8 dense matvec, the scalar form of src/engine/matvec_fp8.inc:42-82 (matvec_dense, ops.cpp:284-289):
 * W row-major [rows x cols] E4M3, one UE8M0 scale per 128x128 tile in S row-major
 * [ceil(rows/128)][ceil(cols/128)]. Per row, each 128-column run is summed on its own (a float
 * chain over the run) and multiplied by its tile's scale into the row sum. */
void orc_matvec_fp8(const uint8_t* w, const uint8_t* s, uint64_t rows, uint64_t cols, const float* x,
                    float* out) {
  const uint64_t sc_cols = (cols + 127) / 128;
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = orc_e4m3_to_float((uint8_t)i);
#pragma omp parallel for schedule(static)
  for (uint64_t r = 0; r < rows; ++r) {
    const uint8_t* wr = w + r * cols;
    const uint8_t* sr = s + (r >> 7) * sc_cols;
    float acc = 0.0f;
    for (uint64_t t = 0; t < sc_cols; ++t) {
      const uint64_t c0 = t * 128, c1 = c0 + 128 < cols ? c0 + 128 : cols;
      float sub = 0.0f;
      for (uint64_t c = c0; c < c1; ++c) sub += lut[wr[c]] * x[c];
      acc += sub * orc_e8m0_to_float(sr[t]);
    }
    out[r] = acc;
  }
}

/* The shared expert on one token, the CPU composition of src/engine/model.cpp:1214-1222: gate and
 * up [inter x hidden] and down [hidden x inter] FP8 dense, sh = W_d . swiglu(W_g x, W_u x), then
 * block[d] += sh[d]. */
void orc_shared_expert(const uint8_t* wg, const uint8_t* sg, const uint8_t* wu, const uint8_t* su,
                       const uint8_t* wd, const uint8_t* sd, uint64_t hidden, uint64_t inter, float limit,
                       const float* x, float* block) {
  float* g = (float*)calloc(inter, sizeof(float));
  float* u = (float*)calloc(inter, sizeof(float));
  float* a = (float*)calloc(inter, sizeof(float));
  float* sh = (float*)calloc(hidden, sizeof(float));
  orc_matvec_fp8(wg, sg, inter, hidden, x, g);
  orc_matvec_fp8(wu, su, inter, hidden, x, u);
  orc_swiglu(g, u, inter, limit, a);
  orc_matvec_fp8(wd, sd, hidden, inter, a, sh);
  for (uint64_t d = 0; d < hidden; ++d) block[d] += sh[d];
  free(g);
  free(u);
  free(a);
  free(sh);
}

/* Hyper-connection expand (src/engine/ops.cpp:470-482): lane dst of the next state is
 * block * post[dst] plus comb[dst + src * n_hc] * residual lane src, summed over src in order;
 * each lane [n_embd] at out_hc + dst * n_embd. */
void orc_hc_expand(float* out_hc, const float* block, const float* residual_hc, const float* post,
                   const float* comb, uint32_t n_embd, uint32_t n_hc) {
  for (uint32_t dst = 0; dst < n_hc; ++dst) {
    float* o = out_hc + (uint64_t)dst * n_embd;
    for (uint32_t d = 0; d < n_embd; ++d) o[d] = block[d] * post[dst];
    for (uint32_t src = 0; src < n_hc; ++src) {
      const float c = comb[dst + src * n_hc];
      const float* r = residual_hc + (uint64_t)src * n_embd;
      for (uint32_t d = 0; d < n_embd; ++d) o[d] += c * r[d];
    }
  }
}

/* A layer without a hyper-connection control adds the block into lane 0 only
 * (src/engine/model.cpp:1237-1238; the device form src/gpu/dense_gpu.hip:1717-1724). */
void orc_hc_add(float* hc, const float* block, uint32_t n_embd) {
  for (uint32_t d = 0; d < n_embd; ++d) hc[d] += block[d];
}

/* ------------------------------------------------------------------------------------------ */
/* the reference's separable batch-pipeline steps                                              */
/* ------------------------------------------------------------------------------------------ */

/* f32 -> E4M3 (OCP fn) to nearest, ties to the even code, for |v| <= 448: the conversion the
 * reference's requantise calls (v_cvt_pk_fp8_f32) on inputs it has clamped to +-448
 * (src/gpu/expert_kernel.hip:913-924). Chooses the nearer of the two neighbouring codes by value,
 * so it follows from the value table alone. */
uint8_t orc_f32_to_e4m3(float v) {
  const float* t = e4m3_table();
  const uint8_t s = signbit(v) ? 0x80 : 0x00;
  const float a = fabsf(v);
  int lo = 0;
  for (int c = 1; c <= 0x7E; ++c)
    if (t[c] <= a) lo = c;
  if (lo == 0x7E) return s | 0x7E;
  const float dl = a - t[lo], dh = t[lo + 1] - a;
  const int c = dl < dh ? lo : dh < dl ? lo + 1 : ((lo & 1) ? lo + 1 : lo);
  return s | (uint8_t)c;
}

/* expert_swiglu_quant_kernel, src/gpu/expert_kernel.hip:862-931: g, u bf16 [dim][total]
 * (dim-major), w f32 [total] or NULL; v = silu(min(g, L)) * clamp(u, -L, L) * w (no clamp when
 * L <= 0, fminf/fmaxf forms), then per (slot, 128-row band) scale = max |v| / 448 (1 when zero),
 * scales [total][dim / 128], out E4M3 [total][dim] = e4m3(clamp(v * (1 / scale), -448, 448)). */
void orc_swiglu_quant(const uint16_t* g, const uint16_t* u, const float* w, uint8_t* out, float* scales,
                      uint32_t dim, uint32_t total, float limit) {
  const uint32_t nkb = dim >> 7;
  float v[128];
  for (uint32_t sl = 0; sl < total; ++sl) {
    const float wv = w ? w[sl] : 1.0f;
    for (uint32_t kb = 0; kb < nkb; ++kb) {
      float m = 0.0f;
      for (uint32_t k = 0; k < 128; ++k) {
        const size_t o = (size_t)(kb * 128 + k) * total + sl;
        float gv = orc_bf16_to_f32(g[o]), uv = orc_bf16_to_f32(u[o]);
        if (limit > 0.0f) {
          gv = fminf(gv, limit);
          uv = fminf(limit, fmaxf(-limit, uv));
        }
        v[k] = (gv / (1.0f + expf(-gv))) * uv * wv;
        m = fmaxf(m, fabsf(v[k]));
      }
      const float sc = m > 0.0f ? m * (1.0f / 448.0f) : 1.0f;
      scales[(size_t)sl * nkb + kb] = sc;
      const float inv = 1.0f / sc;
      for (uint32_t k = 0; k < 128; ++k)
        out[(size_t)sl * dim + kb * 128 + k] = orc_f32_to_e4m3(fminf(fmaxf(v[k] * inv, -448.0f), 448.0f));
    }
  }
}

/* expert_scatter_slots_kernel, src/gpu/expert_kernel.hip:935-947: block[h][t] += (the float sum
 * from zero, in ord order, of bf16 y[h][ord[i]] for i in run[t] .. run[t+1]-1); tokens with an
 * empty run are left as they are. */
void orc_scatter_slots(const uint16_t* y, float* block, const uint32_t* ord, const uint32_t* run, uint32_t dim,
                       uint32_t nb_tok, uint32_t nb_stride, uint32_t total) {
  for (uint32_t h = 0; h < dim; ++h) {
    const uint16_t* row = y + (size_t)h * total;
    for (uint32_t t = 0; t < nb_tok; ++t) {
      const uint32_t a = run[t], b = run[t + 1];
      if (a == b) continue;
      float acc = 0.0f;
      for (uint32_t i = a; i < b; ++i) acc += orc_bf16_to_f32(row[ord[i]]);
      block[(size_t)h * nb_stride + t] += acc;
    }
  }
}

/* expert_gather_tokens_kernel, src/gpu/expert_kernel.hip:828-835: dst[c][t] = src[c][tok[t]]. */
void orc_gather_tokens(const float* src, float* dst, const uint32_t* tok, uint32_t dim, uint32_t nb, uint32_t nt) {
  for (uint32_t c = 0; c < dim; ++c)
    for (uint32_t t = 0; t < nt; ++t) dst[(size_t)c * nt + t] = src[(size_t)c * nb + tok[t]];
}

/* The reference's single-matrix W8A8 GEMM for one tile (expert_gemm_wmma_kernel,
 * src/gpu/expert_kernel.hip:364-825): for row r and column j < nt, t = tok ? tok[j] : j,
 *   out = fold over the 128-column blocks kb in order of fmaf(raw_kb, xs[t][kb], out), raw_kb =
 *         the block's sum of W8[r][k] * x8[t][k] (the products are exact in f32; summed here in
 *         double and rounded once), W8 = the weight's value without its row scale, i.e.
 *         dequantize_matrix (blockquant.cpp:793-833) with rscale 1: 2^s * (+-1) * e[(p + rh) % 4];
 *   y[r * yld + j] = out * (bf16 rscales[r] * wscale) (expert_kernel.hip:808-837), f32 or, with
 *         y_bf16, bf16 by round to nearest even. yld = ld ? ld : nt. Planes in the container's
 *         row-major bit streams; cb the unpacked f32 codebook [2][1024][4]. */
void orc_expert_gemm_w8a8(const uint8_t* codes, const uint8_t* fields, const uint16_t* rscales, const uint32_t* tok,
                          uint32_t nt, uint32_t ld, const uint8_t* x8, const float* xs, const float* cb,
                          uint64_t rows, uint64_t cols, float wscale, int y_bf16, void* y) {
  const uint64_t nblk = cols / ORC_BLOCK, codes_row = cols / 4, nkb = cols / 128;
  const uint32_t yld = ld ? ld : nt;
  float x8f[256];
  for (int i = 0; i < 256; ++i) x8f[i] = orc_e4m3_to_float((uint8_t)i);
#pragma omp parallel for num_threads(NT) schedule(static)
  for (uint64_t r = 0; r < rows; ++r) {
    float* w8 = (float*)malloc(cols * sizeof(float));
    for (uint64_t b = 0; b < nblk; ++b) {
      const uint32_t f = orc_unpack_bits(fields, r * nblk + b, 6);
      const uint32_t s = f & 7u, g = (f >> 3) & 3u;
      const uint32_t v = (f >> 5) < 1u ? (f >> 5) : 1u;
      const float bs = (float)(1u << s) * ((g & 1u) ? -1.0f : 1.0f);
      const uint32_t rh = (g & 2u) ? 2u : 0u;
      for (int i = 0; i < 4; ++i) {
        const uint32_t c = orc_unpack_bits(codes, r * codes_row + b * 4 + i, 10);
        const float* e = cb + ((size_t)v * ORC_LUT + c) * 4;
        for (uint32_t p = 0; p < 4; ++p) w8[b * ORC_BLOCK + i * 4 + p] = bs * e[(p + rh) % 4];
      }
    }
    const float rs = orc_bf16_to_f32(rscales[r]) * wscale;
    for (uint32_t j = 0; j < nt; ++j) {
      const uint32_t t = tok ? tok[j] : j;
      const uint8_t* xr = x8 + (size_t)t * cols;
      float out = 0.0f;
      for (uint64_t kb = 0; kb < nkb; ++kb) {
        double acc = 0.0;
        for (uint64_t k = kb * 128; k < kb * 128 + 128; ++k) acc += (double)w8[k] * (double)x8f[xr[k]];
        out = fmaf((float)acc, xs[(size_t)t * nkb + kb], out);
      }
      const float val = out * rs;
      if (y_bf16)
        ((uint16_t*)y)[r * yld + j] = orc_f32_to_bf16(val);
      else
        ((float*)y)[r * yld + j] = val;
    }
    free(w8);
  }
}
