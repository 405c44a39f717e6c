/*
 * CPU oracle: a C restatement of the reference's CPU path for the 2.875-bpw quad-codebook
 * routed experts (AFF_Q2P875_Q4). TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker. The product (affinity_amd/) never links, imports or calls it.
 *
 * Every function cites the reference file:line it restates (paths under the reference tree).
 * How each one is pinned (golden vectors written by the compiled reference, closed forms,
 * invariants, brute force) is listed in tests/test_oracle.py; none is "parity unpinned".
 *
 * Conventions:
 *  - A matrix is row-major [rows x cols]; its planes are the container's: `codes` is an
 *    LSB-first stream of 10-bit quad codes (rows*cols/4 of them), `fields` an LSB-first stream
 *    of 6-bit block fields (rows*cols/16), `rscales` one bf16 per row.
 *  - A float codebook is float[2 variants][1024 codes][4]; a packed codebook is uint32[2048]
 *    (dword v*1024+c, byte p = E4M3 encoding of element p).
 */
#ifndef AFFX_ORACLE_H
#define AFFX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ORC_BLOCK = 16, ORC_PAIR = 4, ORC_CODE_BITS = 10, ORC_FIELD_BITS = 6, ORC_SCALE_BITS = 3,
  ORC_LUT = 1024, ORC_VARIANTS = 2, ORC_BIAS = 7
};

/* threads used by the parallel loops below (0 = OpenMP default) */
void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- element codecs ---- */
float orc_e4m3_to_float(uint8_t b);
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);

/* ---- bit streams ---- */
void orc_pack_bits(uint8_t* dst, uint64_t index, uint32_t bits, uint32_t value);
uint32_t orc_unpack_bits(const uint8_t* src, uint64_t index, uint32_t bits);

/* ---- synthetic inputs (BASELINE generator: splitmix64 + Box-Muller, bf16 RNE) ---- */
uint64_t orc_splitmix_at(uint64_t seed, uint64_t k);
void orc_gen_normal_bf16(uint64_t seed, uint64_t n, double scale, float* out);
void orc_gen_normal_f64(uint64_t seed, uint64_t n, double* out);

/* ---- container geometry ---- */
uint64_t orc_expert_layout(uint64_t hidden, uint64_t inter, uint64_t* off9, uint64_t* size9);

/* ---- codebook fitting ---- */
uint64_t orc_collect_samples(const float* w, uint64_t rows, uint64_t cols, uint64_t budget,
                             float* out, uint64_t cap);
void orc_fit_codebook(const float* samples, uint64_t n_samples, uint32_t iters, uint64_t seed,
                      float* cb);
uint8_t orc_e4m3_nearest(float x);
void orc_project_codebook(float* cb, uint64_t n);
void orc_pack_codebook(const float* cb, uint32_t* packed);
void orc_unpack_codebook(const uint32_t* packed, float* cb);
int orc_codebook_exponents_ok(const uint32_t* packed);

/* ---- quantise / dequantise one matrix ---- */
int orc_quantize_matrix(const float* w, uint64_t rows, uint64_t cols, const float* cb,
                        const float* col_importance, uint8_t* codes, uint8_t* fields,
                        uint16_t* rscales);
int orc_dequantize_matrix(const uint8_t* codes, const uint8_t* fields, const uint16_t* rscales,
                          uint64_t rows, uint64_t cols, const float* cb, float* out);

/* ---- CPU expert compute ---- */
void orc_expert_gemv(const uint8_t* codes, const uint8_t* fields, const uint16_t* rscales,
                     uint64_t rows, uint64_t cols, const float* cb, const float* x, float w,
                     float* y);
void orc_swiglu(const float* gate, const float* up, uint64_t n, float limit, float* out);
void orc_expert_ffn(const uint8_t* expert, uint64_t hidden, uint64_t inter, const float* cb,
                    const float* x, float w, float limit, float* y);

/* ---- routing ---- */
void orc_route_softmax_topk(const float* logits, uint32_t n_expert, uint32_t k, uint32_t* sel,
                            float* w);
float orc_sqrtsoftplus(float x);
uint32_t orc_route_topk(const float* logits, const float* bias, uint32_t n_expert, uint32_t k,
                        int norm_topk_prob, float routed_scaling, uint32_t* sel, float* w);

/* ---- the step after the routed experts: shared expert and hyper-connection post ---- */
float orc_e8m0_to_float(uint8_t e);
void orc_matvec_fp8(const uint8_t* w, const uint8_t* s, uint64_t rows, uint64_t cols, const float* x,
                    float* out);
void orc_shared_expert(const uint8_t* wg, const uint8_t* sg, const uint8_t* wu, const uint8_t* su,
                       const uint8_t* wd, const uint8_t* sd, uint64_t hidden, uint64_t inter, float limit,
                       const float* x, float* block);
void orc_hc_expand(float* out_hc, const float* block, const float* residual_hc, const float* post,
                   const float* comb, uint32_t n_embd, uint32_t n_hc);
void orc_hc_add(float* hc, const float* block, uint32_t n_embd);

/* ---- the reference's separable batch-pipeline steps ---- */
uint8_t orc_f32_to_e4m3(float v);
void orc_swiglu_quant(const uint16_t* g, const uint16_t* u, const float* w, uint8_t* out, float* scales,
                      uint32_t dim, uint32_t total, float limit);
void orc_scatter_slots(const uint16_t* y, float* block, const uint32_t* ord, const uint32_t* run, uint32_t dim,
                       uint32_t nb_tok, uint32_t nb_stride, uint32_t total);
void orc_gather_tokens(const float* src, float* dst, const uint32_t* tok, uint32_t dim, uint32_t nb, uint32_t nt);
void orc_expert_gemm_w8a8(const uint8_t* codes, const uint8_t* fields, const uint16_t* rscales, const uint32_t* tok,
                          uint32_t nt, uint32_t ld, const uint8_t* x8, const float* xs, const float* cb,
                          uint64_t rows, uint64_t cols, float wscale, int y_bf16, void* y);

#ifdef __cplusplus
}
#endif
#endif
