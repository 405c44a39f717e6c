// C-ABI shim over the reference's own CPU path, compiled together with the reference sources
// from /root/reference by oracle/Makefile into oracle/_ref/libaffref.so.
//
// This file is test infrastructure. It holds no algorithm: every function forwards to the
// reference implementation it names so that tests/golden/make_golden.py (fixture generation),
// the oracle cross-checks in tests/ and bench.py's cpu_baseline leg can call the reference
// through ctypes. The planes use the reference's row-major container layout
// (src/format/aff_format.cpp:45-91); the codebook is float[variant][code][4]
// (src/quant/blockquant.h:87-97).
#include "quant/blockquant.h"
#include "quant/source_dtypes.h"
#include "format/aff_format.h"
#include "engine/expert_kernel.h"
#include "engine/ops.h"
#include "engine/threadpool.h"
#include "format/aff_reader.h"
#include "format/aff_writer.h"

#include <cstring>
#include <vector>

using namespace aff;

namespace {

QuantSpec q4_spec() { return expert_quant_spec((uint32_t)AFF_Q2P875_Q4); }

Codebook codebook_from(const float* cb) {
  const QuantSpec sp = q4_spec();
  Codebook c;
  c.pair = sp.pair;
  c.variants = sp.variants();
  c.k = sp.lut_size();
  c.v.assign(cb, cb + (size_t)c.variants * c.k * c.pair);
  return c;
}

ExpertMatrixView view(const uint8_t* codes, const uint8_t* fields, const uint8_t* rscales,
                      uint64_t rows, uint64_t cols) {
  ExpertMatrixView m;
  m.data = codes;
  m.scales = fields;
  m.rscales = rscales;
  m.rows = rows;
  m.cols = cols;
  m.spec = q4_spec();
  return m;
}

}  // namespace

extern "C" {

// src/quant/blockquant.cpp:386-423
uint64_t affref_collect_samples(const float* w, uint64_t rows, uint64_t cols, uint64_t budget,
                                float* out, uint64_t cap) {
  std::vector<float> s;
  collect_normalized_samples(w, rows, cols, q4_spec(), &s, budget, nullptr, nullptr);
  const uint64_t n = s.size() < cap ? s.size() : cap;
  if (out && n) std::memcpy(out, s.data(), n * sizeof(float));
  return s.size();
}

// src/quant/blockquant.cpp:252-384 (fit) then 463-466 (projection onto E4M3, pow2 constraint),
// the order tools/aff_quantize.cpp:429-434 uses.
void affref_fit_codebook(const float* samples, uint64_t n, uint32_t iters, uint64_t seed,
                         int project, float* cb_out) {
  Codebook cb = fit_codebook(samples, n, q4_spec(), nullptr, iters, seed);
  if (project) project_codebook_e4m3(&cb, true);
  std::memcpy(cb_out, cb.v.data(), cb.v.size() * sizeof(float));
}

// src/quant/blockquant.cpp:468-480
void affref_pack_codebook(const float* cb, uint32_t* packed) {
  const std::vector<uint32_t> p = pack_codebook_e4m3_quads(codebook_from(cb));
  std::memcpy(packed, p.data(), p.size() * sizeof(uint32_t));
}

// src/quant/blockquant.cpp:482-492
void affref_unpack_codebook(const uint32_t* packed, float* cb) {
  const QuantSpec sp = q4_spec();
  Codebook c;
  unpack_codebook_e4m3_quads(packed, sp.variants(), sp.lut_size(), &c);
  std::memcpy(cb, c.v.data(), c.v.size() * sizeof(float));
}

// src/quant/blockquant.cpp:498-556: the acceleration grid aff-quantize builds once per codebook.
void* affref_search_new(const float* cb) {
  CodebookSearch* s = new CodebookSearch;
  build_codebook_search(codebook_from(cb), s);
  return s;
}
void affref_search_free(void* s) { delete static_cast<CodebookSearch*>(s); }

// src/quant/blockquant.cpp:586-791. `search` may be null (plain scan).
int affref_quantize_matrix(const float* w, uint64_t rows, uint64_t cols, const float* cb,
                           const float* col_importance, void* search, uint8_t* codes,
                           uint8_t* fields, uint8_t* rscales) {
  QuantizedMatrix q;
  std::string err;
  if (!quantize_matrix(w, rows, cols, q4_spec(), codebook_from(cb), &q, &err, col_importance,
                       static_cast<CodebookSearch*>(search)))
    return -1;
  std::memcpy(codes, q.data.data(), q.data.size());
  std::memcpy(fields, q.scales.data(), q.scales.size());
  std::memcpy(rscales, q.rscales.data(), q.rscales.size());
  return 0;
}

// src/quant/blockquant.cpp:793-833
int affref_dequantize_matrix(const uint8_t* codes, const uint8_t* fields, const uint8_t* rscales,
                             uint64_t rows, uint64_t cols, const float* cb, float* out) {
  const QuantSpec sp = q4_spec();
  QuantizedMatrix q;
  q.rows = rows;
  q.cols = cols;
  q.spec = sp;
  q.data.assign(codes, codes + rows * cols / sp.pair * sp.code_bits / 8);
  q.scales.assign(fields, fields + rows * (cols / sp.block) * sp.block_field_bits() / 8);
  q.rscales.assign(rscales, rscales + rows * 2);
  std::string err;
  return dequantize_matrix(q, codebook_from(cb), out, &err) ? 0 : -1;
}

// src/engine/expert_kernel.cpp:119-139: y[r] += w * (W x)[r]; mt selects expert_gemv_scaled_mt
// (rows split over the reference's global pool, sized to hardware_concurrency).
void affref_expert_gemv_scaled(const uint8_t* codes, const uint8_t* fields,
                               const uint8_t* rscales, uint64_t rows, uint64_t cols,
                               const float* cb, const float* x, float w, float* y, int mt) {
  const Codebook c = codebook_from(cb);
  const ExpertMatrixView m = view(codes, fields, rscales, rows, cols);
  if (mt) expert_gemv_scaled_mt(m, c, x, w, y);
  else expert_gemv_scaled(m, c, x, w, y);
}

// src/engine/ops.cpp:47-60
void affref_swiglu(const float* gate, const float* up, uint64_t n, float limit, float* out) {
  swiglu(gate, up, n, limit, out);
}

// src/quant/source_dtypes.cpp:91-112, 133 and source_dtypes.h:33-46
float affref_e4m3_to_float(uint8_t b) { return fp8_e4m3_to_float(b); }
uint16_t affref_float_to_bf16(float f) { return float_to_bf16(f); }
float affref_bf16_to_float(uint16_t h) { return bf16_to_float(h); }

// src/format/aff_format.cpp:45-91: offsets and sizes of the nine planes of one expert, in the
// order gate/up/down x data/scale/rscale; returns the stride.
uint64_t affref_expert_layout(uint64_t hidden, uint64_t inter, uint64_t* off9, uint64_t* size9) {
  ExpertGeometry g{hidden, inter, AFF_Q2P875_Q4, AFF_Q2P875_Q4, AFF_Q2P875_Q4};
  AffMatrixDesc d[3];
  const uint64_t stride = compute_expert_layout(g, d[0], d[1], d[2]);
  for (int m = 0; m < 3; ++m) {
    off9[3 * m + 0] = d[m].data_off;   size9[3 * m + 0] = d[m].data_size;
    off9[3 * m + 1] = d[m].scale_off;  size9[3 * m + 1] = d[m].scale_size;
    off9[3 * m + 2] = d[m].rscale_off; size9[3 * m + 2] = d[m].rscale_size;
  }
  return stride;
}

// src/engine/threadpool.cpp:122-131: the pool expert_gemv_scaled_mt runs on (hardware_concurrency)
unsigned affref_pool_threads(void) { return global_pool().size(); }

// src/engine/ops.cpp:62-92 (the engine router). Returns the number of experts chosen.
uint32_t affref_route_topk(const float* logits, const float* bias, uint32_t n_expert, uint32_t top_k,
                           int norm_topk_prob, float routed_scaling, uint32_t* sel, float* w) {
  RouterOut out{};
  route_topk(logits, bias, n_expert, top_k, norm_topk_prob != 0, routed_scaling, &out);
  for (uint32_t i = 0; i < out.n; ++i) { sel[i] = out.expert[i]; w[i] = out.weight[i]; }
  return out.n;
}

// A container through the reference's own writer (src/format/aff_writer.cpp): n_layers layers of
// n_experts quad-format experts (container layout, `stride` bytes each, laid out [layer][expert]
// in `experts`), the packed codebook as the `__codebook` tensor (1 x 2048, f32-declared, the
// bytes of the dwords: tools/aff_quantize.cpp:262-271, 514-527) and one small bf16 tensor.
// Returns 0, or -1 with the writer's message in err.
int affref_write_container(const char* path, const char* meta, uint32_t n_layers, uint32_t n_experts,
                           uint64_t hidden, uint64_t inter, const uint32_t* codebook, const uint8_t* experts,
                           uint64_t stride, char* err, uint64_t err_len) {
  std::vector<LayerDecl> layers(n_layers);
  for (auto& L : layers) {
    L.n_experts = n_experts;
    L.geom = ExpertGeometry{hidden, inter, AFF_Q2P875_Q4, AFF_Q2P875_Q4, AFF_Q2P875_Q4};
  }
  std::vector<TensorDecl> tensors(2);
  tensors[0] = TensorDecl{"__codebook", 1, 2048, AFF_F32};
  tensors[1] = TensorDecl{"blk.0.norm", 1, 64, AFF_BF16};
  AffWriter w;
  std::string e;
  auto fail = [&]() {
    std::snprintf(err, err_len, "%s", e.c_str());
    return -1;
  };
  if (!w.begin(path, meta, layers, tensors, &e)) return fail();
  MatrixData cb;
  cb.data = codebook;
  cb.data_size = 2048 * 4;
  if (!w.write_tensor("__codebook", cb, &e)) return fail();
  std::vector<uint16_t> norm(64, 0x3F80);
  MatrixData nm;
  nm.data = norm.data();
  nm.data_size = 128;
  if (!w.write_tensor("blk.0.norm", nm, &e)) return fail();
  AffMatrixDesc g, u, d;
  compute_expert_layout(ExpertGeometry{hidden, inter, AFF_Q2P875_Q4, AFF_Q2P875_Q4, AFF_Q2P875_Q4}, g, u, d);
  for (uint32_t l = 0; l < n_layers; ++l)
    for (uint32_t x = 0; x < n_experts; ++x) {
      const uint8_t* p = experts + ((uint64_t)l * n_experts + x) * stride;
      auto md = [&](const AffMatrixDesc& m) {
        MatrixData r;
        r.data = p + m.data_off; r.data_size = m.data_size;
        r.scales = p + m.scale_off; r.scale_size = m.scale_size;
        r.rscales = p + m.rscale_off; r.rscale_size = m.rscale_size;
        return r;
      };
      ExpertData ed{md(g), md(u), md(d)};
      if (!w.write_expert(l, x, ed, &e)) return fail();
    }
  if (!w.finalize(&e)) return fail();
  return 0;
}

// The reference reader's addressing (src/format/aff_reader.h:45-48): the file offset of expert
// (layer, expert), or -1 if the file does not open.
int64_t affref_expert_offset(const char* path, uint32_t layer, uint32_t expert) {
  AffReader r;
  std::string e;
  if (!r.open(path, &e)) return -1;
  const uint8_t* base = r.expert_ptr(0, 0) - r.header().expert_pool_off - r.layer(0).base_off;
  return (int64_t)(r.expert_ptr(layer, expert) - base);
}

// src/engine/ops.cpp:284-289 -> src/engine/matvec_fp8.inc:42-82: the FP8 dense matvec (E4M3
// weights, one UE8M0 scale per 128x128 tile), single-threaded.
void affref_matvec_fp8(const uint8_t* w, const uint8_t* s, uint64_t rows, uint64_t cols, const float* x,
                       float* out) {
  DenseW d;
  d.data = w;
  d.scales = s;
  d.quant = AFF_FP8_E4M3;
  matvec_dense(d, x, rows, cols, out);
}

// src/quant/source_dtypes.cpp:41-53
float affref_e8m0_to_float(uint8_t e) { return e8m0_to_float(e); }

// src/engine/ops.cpp:470-482
void affref_hc_expand(float* out_hc, const float* block, const float* residual_hc, const float* post,
                      const float* comb, uint32_t n_embd, uint32_t n_hc) {
  hc_expand(out_hc, block, residual_hc, post, comb, n_embd, n_hc);
}

}  // extern "C"
