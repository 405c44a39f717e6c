// Runs libaffx's kernels on the CPU (see hip/hip_runtime.h) against the C oracle.
// Test infrastructure: built with AddressSanitizer by tests/test_cpu_emulation.py.
//
//   emu_main decode  hidden inter n_experts M K seed [staged|allpad|dm<nb>] -> rel_l2 of the decode FFN (the
//                    fused launch, also checked equal to the staged launches; `staged` alone)
//   emu_main grouped hidden inter n_experts T K seed lo   -> rel_l2 of the grouped FFN
//   emu_main quant   rows cols seed                       -> planes bit-exact vs the oracle
//   emu_main dequant hidden inter seed                    -> dequant bit-exact vs the oracle
//   emu_main slots   hidden inter n_experts T K seed      -> the slot-list grouped entry vs the
//                    routes entry (bit for bit) and, with a reordered list, vs the oracle
//   emu_main ffnptr  hidden inter n_experts seed          -> affx_expert_ffn (pointer table) vs
//                    the staged decode (bit for bit) and the oracle
//   emu_main route   n_tok n_experts top_k seed           -> the device router vs the oracle's
//   emu_main shared  hidden inter M T seed                -> the shared expert (decode on M
//                    tokens, batch on T with and without a low part) vs the oracle, and the
//                    hyper-connection post (single and batch forms) bit for bit
//   emu_main fit     rows cols budget iters seed [seq]    -> sample collection, the codebook fit
//                    (with `seq` every k-means++ draw by the sequential sums), projection, packing
//                    and unpacking, each bit for bit vs the oracle
//   emu_main w8a8    hidden inter seed                    -> the single-matrix W8A8 GEMM (three
//                    tiles, f32 and bf16 outputs, a strided arena) vs the oracle
//   emu_main timeout hidden inter n_experts M K seed      -> a decode whose waiters give up (spin
//                    limit 0 from the host) fails the engine hook and affx_decode_status; after
//                    the reset, the next calls are correct
//
// Exit status 0 when the check passes.
#include <hip/hip_runtime.h>

thread_local emu_dim3 threadIdx, blockIdx;
emu_dim3 blockDim, gridDim;
thread_local EmuBlock* emu_blk;

#include "../../affinity_amd/csrc/affx_common.h"
using namespace affx;

extern "C" {
#include "../../oracle/oracle.h"
}

#include <algorithm>
#include <random>
#include <string>

// The library GEMM of affx_blas.cpp (hipBLASLt on the device) as a plain loop with the same
// contract: D[n][m] = sum_k A[m][k] B[n][k] (+ D[n][m]), bf16 operands, products summed in double.
namespace affx {
int blas_gemm_bf16_nt(uint32_t M, uint32_t N, uint32_t K, const void* A, uint32_t lda, const void* B, uint32_t ldb,
                      float* D, uint32_t ldd, int beta_one, hipStream_t) {
  const uint16_t* a = (const uint16_t*)A;
  const uint16_t* b = (const uint16_t*)B;
  auto wide = [](uint16_t v) {
    const uint32_t u = (uint32_t)v << 16;
    float r;
    memcpy(&r, &u, 4);
    return (double)r;
  };
  for (uint32_t n = 0; n < N; ++n)
    for (uint32_t m = 0; m < M; ++m) {
      double acc = beta_one ? (double)D[(size_t)n * ldd + m] : 0.0;
      for (uint32_t k = 0; k < K; ++k) acc += wide(a[(size_t)m * lda + k]) * wide(b[(size_t)n * ldb + k]);
      D[(size_t)n * ldd + m] = (float)acc;
    }
  return 0;
}
}  // namespace affx

namespace {

constexpr uint32_t kCbFloats = kVariants * kLut * 4;  // a codebook as floats [2][1024][4]

uint16_t bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFF + ((u >> 16) & 1)) >> 16);
}

std::vector<uint32_t> load_codebook() {
  std::vector<uint32_t> cb(2048);
  FILE* f = fopen("tests/golden/c1_codebook.bin", "rb");
  if (!f || fread(cb.data(), 4, 2048, f) != 2048) { fprintf(stderr, "codebook fixture missing\n"); exit(2); }
  fclose(f);
  return cb;
}

// Random planes (every field value) with bf16 row scales in [4e-4, 2e-3).
void random_expert(std::mt19937_64& rng, uint8_t* ex, const uint64_t* off, const uint64_t* size) {
  for (int p = 0; p < 9; ++p) {
    if (p % 3 == 2) {
      for (uint64_t r = 0; r < size[p] / 2; ++r) {
        const uint16_t h = bf16(4e-4f + 1.6e-3f * (float)(rng() % 1000) / 1000.f);
        memcpy(ex + off[p] + 2 * r, &h, 2);
      }
    } else {
      for (uint64_t i = 0; i < size[p]; ++i) ex[off[p] + i] = rng() & 0xff;
    }
  }
}

double rel_l2(const std::vector<float>& a, const std::vector<float>& b) {
  double num = 0, den = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    num += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
    den += (double)b[i] * b[i];
  }
  return den > 0 ? sqrt(num / den) : sqrt(num);
}

struct Layer {
  uint32_t hidden, inter, n;
  uint64_t stride, off[9], size[9];
  std::vector<uint8_t> cont, dev;
  std::vector<uint32_t> cb;
  std::vector<float> cbf;
  Layer(uint32_t h, uint32_t i, uint32_t n_, std::mt19937_64& rng) : hidden(h), inter(i), n(n_) {
    stride = affx_expert_layout(h, i, off, size);
    cont.assign(n * stride, 0);
    dev.assign(n * stride, 0);
    for (uint32_t e = 0; e < n; ++e) {
      random_expert(rng, cont.data() + e * stride, off, size);
      if (affx_expert_to_device_layout(cont.data() + e * stride, dev.data() + e * stride, h, i)) exit(3);
    }
    cb = load_codebook();
    cbf.assign(8192, 0.f);
    orc_unpack_codebook(cb.data(), cbf.data());
  }
  affx_layer abi() { return affx_layer{dev.data(), stride, n, hidden, inter, cb.data(), 10.0f}; }
  void oracle(const float* x, const uint32_t* sel, const float* w, uint32_t T, uint32_t K, float* y) {
    for (uint32_t t = 0; t < T; ++t)
      for (uint32_t j = 0; j < K; ++j) {
        const uint32_t e = sel[t * K + j];
        if (e >= n) continue;
        orc_expert_ffn(cont.data() + (uint64_t)e * stride, hidden, inter, cbf.data(), x + (uint64_t)t * hidden,
                       w[t * K + j], 10.0f, y + (uint64_t)t * hidden);
      }
  }
};

void routes(std::mt19937_64& rng, uint32_t T, uint32_t K, uint32_t n, std::vector<uint32_t>& sel,
            std::vector<float>& w) {
  sel.resize(T * K);
  w.resize(T * K);
  std::vector<uint32_t> ids(n);
  for (uint32_t t = 0; t < T; ++t) {
    for (uint32_t i = 0; i < n; ++i) ids[i] = i;
    std::shuffle(ids.begin(), ids.end(), rng);
    for (uint32_t j = 0; j < K; ++j) {
      sel[t * K + j] = ids[j % n];
      w[t * K + j] = 0.05f + (float)(rng() % 1000) / 1000.f;
    }
  }
}

int run_decode(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]), n = atoi(argv[4]), M = atoi(argv[5]),
                 K = atoi(argv[6]);
  std::mt19937_64 rng(atoi(argv[7]));
  Layer L(hidden, inter, n, rng);
  std::vector<float> x(M * hidden), y(M * hidden, 0.f), yref(M * hidden, 0.f), w;
  std::vector<uint32_t> sel;
  std::normal_distribution<float> nd;
  for (auto& v : x) v = 0.5f * nd(rng);
  routes(rng, M, K, n, sel, w);
  if (M > 1) sel[K - 1] = n + 7;  // a padding id
  const std::string mode = argc > 8 ? argv[8] : "";
  if (mode == "allpad")  // no route names an expert of the layer: y = 0
    for (auto& s : sel) s = n + 7;
  affx_layer abi = L.abi();
  const bool staged_only = mode == "staged";
  const size_t wsb = affx_decode_workspace_size(M, K, hidden, inter);
  std::vector<uint8_t> ws(wsb, 0), ws2(wsb, 0);
  std::vector<float> y2(M * hidden, 0.f);
  int rc = affx_decode_staged(&abi, x.data(), hidden, 1, M, sel.data(), w.data(), K, y2.data(), hidden, 1, 0,
                              ws2.data(), wsb, nullptr);
  bool same = true;
  if (!staged_only && rc == 0) {
    // twice on one workspace: the second launch relies on the first leaving its counters zero
    // "dm<nb>": x as the engine's dim-major arena [hidden][nb] (tok stride 1, dim stride nb), the
    // unused token slots of each row filled with huge values that must not reach the result
    const uint32_t nb = mode.rfind("dm", 0) == 0 ? (uint32_t)atoi(mode.c_str() + 2) : 0;
    std::vector<float> xd(nb ? (size_t)hidden * nb : 0, 3e37f);
    for (uint32_t h = 0; nb && h < hidden; ++h)
      for (uint32_t t = 0; t < M; ++t) xd[(size_t)h * nb + t] = x[(size_t)t * hidden + h];
    for (int rep = 0; rep < 2 && rc == 0; ++rep)
      rc = nb ? affx_expert_ffn_decode(&abi, xd.data(), 1, nb, M, sel.data(), w.data(), K, y.data(), hidden, 1, 0,
                                       ws.data(), wsb, nullptr)
              : affx_expert_ffn_decode(&abi, x.data(), hidden, 1, M, sel.data(), w.data(), K, y.data(), hidden, 1, 0,
                                       ws.data(), wsb, nullptr);
    // the sync run's counter, error bits and release flags are zero again (the one-pass kernel's
    // epoch and publish flags advance from launch to launch)
    uint32_t sync[3];
    memcpy(sync, ws.data(), sizeof(sync));
    uint32_t nonzero = 0;
    for (size_t i = 0; i < kSyncRunBytes; ++i) nonzero += ws[i] != 0 && i / 4 != kEpochWord;
    same = memcmp(y.data(), y2.data(), y.size() * 4) == 0 && nonzero == 0;
    printf("fused: identical to staged=%d counters=%u,%u,%u nonzero_sync_bytes=%u\n", (int)same, sync[0], sync[1],
           sync[2], nonzero);
  } else {
    y = y2;
  }
  L.oracle(x.data(), sel.data(), w.data(), M, K, yref.data());
  double e = 0.0;
  if (mode == "allpad") {
    for (float v : y) e += v != 0.f;  // count of nonzero outputs
  } else {
    e = rel_l2(y, yref);
  }
  printf("decode rc=%d rel_l2=%.3e %s\n", rc, e, rc ? affx_last_error() : "");
  return rc == 0 && same && e <= 1e-3 ? 0 : 1;
}

int run_grouped(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]), n = atoi(argv[4]), T = atoi(argv[5]),
                 K = atoi(argv[6]);
  std::mt19937_64 rng(atoi(argv[7]));
  const bool lo = argc > 8 && atoi(argv[8]);
  Layer L(hidden, inter, n, rng);
  std::vector<uint16_t> xb(T * hidden), xl(T * hidden);
  std::vector<float> x(T * hidden), y(T * hidden, 0.f), yref(T * hidden, 0.f), w;
  std::vector<uint32_t> sel;
  std::normal_distribution<float> nd;
  for (size_t i = 0; i < x.size(); ++i) {
    const float v = nd(rng);
    xb[i] = bf16(v);
    const float hi = __uint_as_float((uint32_t)xb[i] << 16);
    xl[i] = bf16(v - hi);
    x[i] = lo ? hi + __uint_as_float((uint32_t)xl[i] << 16) : hi;
  }
  routes(rng, T, K, n, sel, w);
  sel[K] = n + 1;  // a padding id
  affx_layer abi = L.abi();
  const size_t wsb = affx_grouped_workspace_size(T, K, n, hidden, inter);
  std::vector<uint8_t> ws(wsb);
  const int rc = affx_expert_ffn_grouped(&abi, xb.data(), lo ? xl.data() : nullptr, T, sel.data(), w.data(),
                                         K, y.data(), 0, ws.data(), wsb, nullptr);
  L.oracle(x.data(), sel.data(), w.data(), T, K, yref.data());
  const double e = rel_l2(y, yref);
  printf("grouped rc=%d rel_l2=%.3e %s\n", rc, e, affx_last_error());
  return rc == 0 && e <= 1e-3 ? 0 : 1;
}

// The slot-list entry: the host builds the list the routes entry builds on the device (slots
// sorted by expert, a token's slots in route order): bit-identical to the routes entry; then the
// same list with each expert's tokens and each token's slots reversed (another valid list): the
// oracle's tolerance.
int run_slots(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]), n = atoi(argv[4]), T = atoi(argv[5]),
                 K = atoi(argv[6]);
  std::mt19937_64 rng(atoi(argv[7]));
  Layer L(hidden, inter, n, rng);
  std::vector<uint16_t> xb(T * hidden);
  std::vector<float> x(T * hidden), y1(T * hidden, 0.f), y2(T * hidden, 0.f), y3(T * hidden, 0.f),
      yref(T * hidden, 0.f), w;
  std::vector<uint32_t> sel;
  std::normal_distribution<float> nd;
  for (size_t i = 0; i < x.size(); ++i) {
    xb[i] = bf16(nd(rng));
    x[i] = __uint_as_float((uint32_t)xb[i] << 16);
  }
  routes(rng, T, K, n, sel, w);
  sel[K + 1] = n + 3;  // a padding id
  affx_layer abi = L.abi();
  const size_t wsb = affx_grouped_workspace_size(T, K, n, hidden, inter);
  std::vector<uint8_t> ws(wsb);
  int rc = affx_expert_ffn_grouped(&abi, xb.data(), nullptr, T, sel.data(), w.data(), K, y1.data(), 0, ws.data(),
                                   wsb, nullptr);
  // the canonical list
  std::vector<uint32_t> start(n + 1, 0), tok, ord, run(T + 1, 0), slot_of(T * K, ~0u);
  std::vector<float> wt;
  for (uint32_t e = 0; e < n; ++e) {
    start[e] = (uint32_t)tok.size();
    for (uint32_t i = 0; i < T * K; ++i)
      if (sel[i] == e) { slot_of[i] = (uint32_t)tok.size(); tok.push_back(i / K); wt.push_back(w[i]); }
  }
  start[n] = (uint32_t)tok.size();
  for (uint32_t t = 0; t < T; ++t) {
    run[t] = (uint32_t)ord.size();
    for (uint32_t j = 0; j < K; ++j)
      if (slot_of[t * K + j] != ~0u) ord.push_back(slot_of[t * K + j]);
  }
  run[T] = (uint32_t)ord.size();
  const uint32_t ns = (uint32_t)tok.size();
  if (rc == 0)
    rc = affx_expert_ffn_grouped_slots(&abi, xb.data(), nullptr, T, start.data(), tok.data(), wt.data(), ord.data(),
                                       run.data(), ns, y2.data(), 0, ws.data(), wsb, nullptr);
  const bool same = memcmp(y1.data(), y2.data(), y1.size() * 4) == 0;
  // another valid list: each expert's slots in reverse token order, each token's slots reversed
  std::vector<uint32_t> tok2(ns), ord2(ns), remap(ns);
  std::vector<float> wt2(ns);
  for (uint32_t e = 0; e < n; ++e)
    for (uint32_t s0 = start[e]; s0 < start[e + 1]; ++s0) {
      const uint32_t s1 = start[e] + start[e + 1] - 1 - s0;
      remap[s0] = s1;
      tok2[s1] = tok[s0];
      wt2[s1] = wt[s0];
    }
  for (uint32_t t = 0; t < T; ++t)
    for (uint32_t i = run[t]; i < run[t + 1]; ++i) ord2[run[t] + run[t + 1] - 1 - i] = remap[ord[i]];
  if (rc == 0)
    rc = affx_expert_ffn_grouped_slots(&abi, xb.data(), nullptr, T, start.data(), tok2.data(), wt2.data(),
                                       ord2.data(), run.data(), ns, y3.data(), 0, ws.data(), wsb, nullptr);
  L.oracle(x.data(), sel.data(), w.data(), T, K, yref.data());
  const double e1 = rel_l2(y1, yref), e3 = rel_l2(y3, yref);
  printf("slots rc=%d slots=%u routes==slots=%d rel_l2 routes=%.3e reordered=%.3e %s\n", rc, ns, (int)same, e1, e3,
         rc ? affx_last_error() : "");
  return rc == 0 && same && e1 <= 1e-3 && e3 <= 1e-3 ? 0 : 1;
}

// affx_expert_ffn (expert_ffn_hip's arguments): each matrix in a buffer of its own, permuted by
// affx_matrix_to_device_layout; bit-identical to the staged decode over a slab of the same experts.
int run_ffnptr(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]), n = atoi(argv[4]);
  std::mt19937_64 rng(atoi(argv[5]));
  Layer L(hidden, inter, n, rng);
  std::vector<std::vector<uint8_t>> bufs;
  bufs.reserve(9 * n);  // references into it are held while it fills
  std::vector<affx_device_expert> des(n);
  for (uint32_t k = 0; k < n; ++k) {
    for (int i = 0; i < 3; ++i) {
      const uint32_t rows = i < 2 ? inter : hidden, cols = i < 2 ? hidden : inter;
      const uint8_t* ex = L.cont.data() + (uint64_t)k * L.stride;
      bufs.emplace_back(L.size[3 * i]);
      std::vector<uint8_t>& c = bufs.back();
      bufs.emplace_back(L.size[3 * i + 1]);
      std::vector<uint8_t>& f = bufs.back();
      bufs.emplace_back(ex + L.off[3 * i + 2], ex + L.off[3 * i + 2] + L.size[3 * i + 2]);
      if (affx_matrix_to_device_layout(ex + L.off[3 * i], ex + L.off[3 * i + 1], c.data(), f.data(), rows, cols))
        return 3;
    }
  }
  for (uint32_t k = 0; k < n; ++k) {
    affx_matrix* m[3] = {&des[k].gate, &des[k].up, &des[k].down};
    for (int i = 0; i < 3; ++i) {
      const uint32_t rows = i < 2 ? inter : hidden, cols = i < 2 ? hidden : inter;
      const size_t b = (size_t)(k * 3 + i) * 3;
      *m[i] = affx_matrix{bufs[b].data(), bufs[b + 1].data(), bufs[b + 2].data(), rows, cols};
    }
  }
  std::vector<float> x(hidden), w(n), y(hidden), ys(hidden), yref(hidden, 0.f);
  std::vector<uint32_t> sel(n);
  std::normal_distribution<float> nd;
  for (auto& v : x) v = nd(rng);
  for (uint32_t k = 0; k < n; ++k) { w[k] = 0.1f + 0.13f * k; sel[k] = k; }
  for (uint32_t h = 0; h < hidden; ++h) y[h] = ys[h] = yref[h] = 0.25f * nd(rng);
  std::vector<float> scratch(2 * n * inter, 1e30f);
  int rc = affx_expert_ffn(des.data(), w.data(), n, L.cb.data(), x.data(), 10.0f, scratch.data(), y.data(), nullptr);
  affx_layer abi = L.abi();
  const size_t wsb = affx_decode_workspace_size(1, n, hidden, inter);
  std::vector<uint8_t> ws(wsb, 0);
  if (rc == 0)
    rc = affx_decode_staged(&abi, x.data(), hidden, 1, 1, sel.data(), w.data(), n, ys.data(), hidden, 1, 1, ws.data(),
                            wsb, nullptr);
  L.oracle(x.data(), sel.data(), w.data(), 1, n, yref.data());
  const bool same = memcmp(y.data(), ys.data(), y.size() * 4) == 0;
  const double e = rel_l2(y, yref);
  printf("ffnptr rc=%d identical to staged=%d rel_l2=%.3e %s\n", rc, (int)same, e, rc ? affx_last_error() : "");
  return rc == 0 && same && e <= 1e-3 ? 0 : 1;
}

// The single-matrix GEMV entries against the oracle's GEMV: every down matrix of n experts (rows
// hidden, cols inter) through affx_expert_gemv_batch with per-matrix weights, and the first one
// through affx_expert_gemv with a host weight, both accumulating into a nonzero y.
int run_gemv(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]), n = atoi(argv[4]);
  std::mt19937_64 rng(atoi(argv[5]));
  Layer L(hidden, inter, n, rng);
  std::vector<affx_matrix> mats(n);
  for (uint32_t k = 0; k < n; ++k) {
    const uint8_t* d = L.dev.data() + (uint64_t)k * L.stride;
    mats[k] = affx_matrix{d + L.off[6], d + L.off[7], d + L.off[8], hidden, inter};
  }
  std::normal_distribution<float> nd;
  std::vector<float> x(inter), w(n), y(hidden), yref(hidden), y1(hidden), y1ref(hidden);
  for (auto& v : x) v = nd(rng);
  for (uint32_t k = 0; k < n; ++k) w[k] = 0.2f + 0.11f * k;
  for (uint32_t h = 0; h < hidden; ++h) y[h] = yref[h] = y1[h] = y1ref[h] = 0.1f * nd(rng);
  int rc = affx_expert_gemv_batch(mats.data(), w.data(), n, L.cb.data(), x.data(), y.data(), nullptr);
  if (rc == 0) rc = affx_expert_gemv(&mats[0], L.cb.data(), x.data(), 0.75f, y1.data(), nullptr);
  for (uint32_t k = 0; k < n; ++k) {
    const uint8_t* ex = L.cont.data() + (uint64_t)k * L.stride;
    orc_expert_gemv(ex + L.off[6], ex + L.off[7], (const uint16_t*)(ex + L.off[8]), hidden, inter, L.cbf.data(),
                    x.data(), w[k], yref.data());
    if (k == 0)
      orc_expert_gemv(ex + L.off[6], ex + L.off[7], (const uint16_t*)(ex + L.off[8]), hidden, inter, L.cbf.data(),
                      x.data(), 0.75f, y1ref.data());
  }
  const double e = rel_l2(y, yref), e1 = rel_l2(y1, y1ref);
  printf("gemv rc=%d batch rel_l2=%.3e single rel_l2=%.3e %s\n", rc, e, e1, rc ? affx_last_error() : "");
  return rc == 0 && e <= 1e-3 && e1 <= 1e-3 ? 0 : 1;
}

// The single-matrix W8A8 GEMM against the oracle: one launch of three tiles (each a different
// expert's down matrix: 64 tokens by identity into a compact block, 13 listed tokens into a strided
// arena, a pad), then a bf16 launch of 5 tokens; the other columns of the strided arena untouched.
int run_w8a8(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]);
  std::mt19937_64 rng(atoi(argv[4]));
  Layer L(hidden, inter, 3, rng);
  const uint32_t rows = hidden, cols = inter, nkb = cols / 128, ntok = 80;
  std::vector<uint8_t> x8((size_t)ntok * cols);
  for (auto& b : x8) {
    b = (uint8_t)(rng() & 0xFF);
    if ((b & 0x7F) == 0x7F) b ^= 1;
  }
  std::uniform_real_distribution<float> ud(0.01f, 2.0f);
  std::vector<float> xs((size_t)ntok * nkb);
  for (auto& v : xs) v = ud(rng);
  std::vector<uint32_t> tok1(13);
  for (auto& t : tok1) t = (uint32_t)(rng() % ntok);
  const uint32_t ld1 = 20;
  std::vector<float> y0((size_t)rows * 64, -1.f), y1((size_t)rows * ld1, 5.f), r0(y0.size()), r1(y1);
  std::vector<uint16_t> yb((size_t)rows * 5), rb(yb.size());
  auto tile = [&](uint32_t e, const uint32_t* tok, void* y, uint32_t nt, uint32_t ld) {
    const uint8_t* d = L.dev.data() + (uint64_t)e * L.stride;
    return affx_expert_tile{d + L.off[6], d + L.off[7], d + L.off[8], tok, y, nt, ld};
  };
  auto oracle = [&](uint32_t e, const uint32_t* tok, void* y, uint32_t nt, uint32_t ld, int bf) {
    const uint8_t* c = L.cont.data() + (uint64_t)e * L.stride;
    orc_expert_gemm_w8a8(c + L.off[6], c + L.off[7], (const uint16_t*)(c + L.off[8]), tok, nt, ld, x8.data(),
                         xs.data(), L.cbf.data(), rows, cols, 0.5f, bf, y);
  };
  affx_expert_tile t3[3] = {tile(0, nullptr, y0.data(), 64, 0), tile(1, tok1.data(), y1.data(), 13, ld1),
                            tile(2, nullptr, nullptr, 0, 0)};
  int rc = affx_expert_gemm_w8a8(t3, 3, 64, x8.data(), xs.data(), L.cb.data(), rows, cols, 0.5f, 0, nullptr);
  affx_expert_tile tb = tile(2, tok1.data() + 3, yb.data(), 5, 0);
  if (rc == 0) rc = affx_expert_gemm_w8a8(&tb, 1, 5, x8.data(), xs.data(), L.cb.data(), rows, cols, 0.5f, 1, nullptr);
  oracle(0, nullptr, r0.data(), 64, 0, 0);
  oracle(1, tok1.data(), r1.data(), 13, ld1, 0);
  oracle(2, tok1.data() + 3, rb.data(), 5, 0, 1);
  // the worst error over each output's scale (its largest magnitude), and the relative L2
  bool ok = rc == 0;
  double num = 0.0, den = 0.0, emax = 0.0, rmax = 0.0;
  for (size_t i = 0; i < y0.size(); ++i) {
    num += (y0[i] - r0[i]) * (double)(y0[i] - r0[i]);
    den += (double)r0[i] * r0[i];
    emax = std::max(emax, (double)std::fabs(y0[i] - r0[i]));
    rmax = std::max(rmax, (double)std::fabs(r0[i]));
  }
  for (size_t i = 0; i < y1.size(); ++i) {
    if (i % ld1 >= 13) {
      ok = ok && y1[i] == 5.f;
      continue;
    }
    num += (y1[i] - r1[i]) * (double)(y1[i] - r1[i]);
    den += (double)r1[i] * r1[i];
    emax = std::max(emax, (double)std::fabs(y1[i] - r1[i]));
    rmax = std::max(rmax, (double)std::fabs(r1[i]));
  }
  const double worst = emax / rmax, l2 = std::sqrt(num / den);
  int bf_off = 0;
  for (size_t i = 0; i < yb.size(); ++i) bf_off = std::max(bf_off, std::abs((int)(int16_t)yb[i] - (int)(int16_t)rb[i]));
  printf("w8a8 rc=%d rel_l2=%.3e worst/max=%.3e bf16_ulps=%d others_kept=%d %s\n", rc, l2, worst, bf_off, (int)ok,
         rc ? affx_last_error() : "");
  return ok && l2 <= 1e-5 && worst <= 1e-5 && bf_off <= 1 ? 0 : 1;
}

// The separable batch-pipeline steps against the oracle: gather and scatter bit for bit, the
// SwiGLU requantise with equal scales and bytes (the emulation's expf is the oracle's).
int run_steps(int argc, char** argv) {
  const uint32_t dim = atoi(argv[2]), nb_tok = atoi(argv[3]);
  std::mt19937_64 rng(atoi(argv[4]));
  std::normal_distribution<float> nd;
  // gather
  const uint32_t nb = nb_tok + 3, nt = nb_tok / 2 + 1;
  std::vector<float> src((size_t)dim * nb), dst((size_t)dim * nt, -1.f), dref((size_t)dim * nt);
  std::vector<uint32_t> tok(nt);
  for (auto& v : src) v = nd(rng);
  for (auto& t : tok) t = rng() % nb;
  int rc = affx_expert_gather_tokens(src.data(), dst.data(), tok.data(), dim, nb, nt, nullptr);
  orc_gather_tokens(src.data(), dref.data(), tok.data(), dim, nb, nt);
  bool ok = rc == 0 && memcmp(dst.data(), dref.data(), dst.size() * 4) == 0;
  // scatter
  std::vector<uint32_t> run(nb_tok + 1, 0);
  for (uint32_t t = 0; t < nb_tok; ++t) run[t + 1] = run[t] + (t == 1 ? 0 : (uint32_t)(rng() % 5));
  const uint32_t total = run[nb_tok];
  std::vector<uint32_t> ordv(total);
  for (uint32_t i = 0; i < total; ++i) ordv[i] = i;
  std::shuffle(ordv.begin(), ordv.end(), rng);
  std::vector<uint16_t> y((size_t)dim * total);
  for (auto& v : y) v = bf16(nd(rng));
  std::vector<float> blk((size_t)dim * nb), bref;
  for (auto& v : blk) v = nd(rng);
  bref = blk;
  if (rc == 0) rc = affx_expert_scatter_slots(y.data(), blk.data(), ordv.data(), run.data(), dim, nb_tok, nb, total, nullptr);
  orc_scatter_slots(y.data(), bref.data(), ordv.data(), run.data(), dim, nb_tok, nb, total);
  ok = ok && rc == 0 && memcmp(blk.data(), bref.data(), blk.size() * 4) == 0;
  // swiglu + requantise over the slot arena
  std::vector<uint16_t> g((size_t)dim * total), u((size_t)dim * total);
  for (auto& v : g) v = bf16(2.5f * nd(rng));
  for (auto& v : u) v = bf16(2.5f * nd(rng));
  std::vector<float> w(total), sc((size_t)total * (dim / 128)), scr(sc.size());
  for (auto& v : w) v = 0.05f + (float)(rng() % 1000) / 1000.f;
  std::vector<uint8_t> out((size_t)total * dim), outr(out.size());
  if (rc == 0) rc = affx_expert_swiglu_quant(g.data(), u.data(), w.data(), out.data(), sc.data(), dim, total, 10.f, nullptr);
  orc_swiglu_quant(g.data(), u.data(), w.data(), outr.data(), scr.data(), dim, total, 10.f);
  ok = ok && rc == 0 && memcmp(out.data(), outr.data(), out.size()) == 0 && memcmp(sc.data(), scr.data(), sc.size() * 4) == 0;
  printf("steps rc=%d total=%u equal=%d %s\n", rc, total, (int)ok, rc ? affx_last_error() : "");
  return ok ? 0 : 1;
}

// The device router against the oracle's: token-major and dim-major logits, both rules, a
// non-multiple-of-64 expert count; ids equal, weights within 2 ulp.
int run_route(int argc, char** argv) {
  const uint32_t T = atoi(argv[2]), E = atoi(argv[3]), K = atoi(argv[4]);
  std::mt19937_64 rng(atoi(argv[5]));
  std::normal_distribution<float> nd;
  std::vector<float> lg(T * E), lgd(T * E), bias(E);
  for (auto& v : lg) v = 2.0f * nd(rng);
  for (auto& v : bias) v = 0.1f * nd(rng);
  for (uint32_t t = 0; t < T; ++t)
    for (uint32_t e = 0; e < E; ++e) lgd[(size_t)e * T + t] = lg[(size_t)t * E + e];
  lg[3] = lg[7] = 50.0f;  // token 0: two tied past the softplus guard
  lgd[3 * T] = lgd[7 * T] = 50.0f;
  bool ok = true;
  int worst = 0;
  for (int rule = 0; rule < 2; ++rule)
    for (int dm = 0; dm < 2; ++dm) {
      std::vector<uint32_t> sel(T * K);
      std::vector<float> w(T * K);
      const int rc = dm ? affx_route_topk(lgd.data(), 1, T, bias.data(), T, E, K, rule, 1, 1.5f, sel.data(), w.data(), nullptr)
                        : affx_route_topk(lg.data(), E, 1, bias.data(), T, E, K, rule, 1, 1.5f, sel.data(), w.data(), nullptr);
      ok = ok && rc == 0;
      for (uint32_t t = 0; t < T; ++t) {
        uint32_t rs[16];
        float rw[16];
        if (rule == AFFX_ROUTE_ENGINE) orc_route_topk(lg.data() + (size_t)t * E, bias.data(), E, K, 1, 1.5f, rs, rw);
        else orc_route_softmax_topk(lg.data() + (size_t)t * E, E, K, rs, rw);
        for (uint32_t j = 0; j < K; ++j) {
          int32_t a, b;
          memcpy(&a, &w[t * K + j], 4);
          memcpy(&b, &rw[j], 4);
          worst = std::max(worst, std::abs(a - b));
          ok = ok && sel[t * K + j] == rs[j];
        }
      }
    }
  printf("route ids equal=%d worst weight ulp=%d\n", (int)ok, worst);
  return ok && worst <= 2 ? 0 : 1;
}

// E4M3 weights that are never NaN (0x7F / 0xFF), UE8M0 tile scales around 2^-7
void fp8_matrix(std::mt19937_64& rng, uint64_t rows, uint64_t cols, std::vector<uint8_t>& w, std::vector<uint8_t>& s) {
  w.resize(rows * cols);
  for (auto& b : w) {
    b = rng() & 0xff;
    if ((b & 0x7f) == 0x7f) b ^= 1;
  }
  s.resize(((rows + 127) / 128) * ((cols + 127) / 128));
  for (auto& e : s) e = (uint8_t)(116 + rng() % 8);
}

int run_shared(int argc, char** argv) {
  const uint32_t H = atoi(argv[2]), I = atoi(argv[3]), M = atoi(argv[4]), T = atoi(argv[5]);
  std::mt19937_64 rng(atoi(argv[6]));
  std::normal_distribution<float> nd;
  std::vector<uint8_t> w[3], sc[3];
  fp8_matrix(rng, I, H, w[0], sc[0]);
  fp8_matrix(rng, I, H, w[1], sc[1]);
  fp8_matrix(rng, H, I, w[2], sc[2]);
  // the kernels read the device layout; the oracle the row-major bytes
  std::vector<uint8_t> wd[3];
  for (int i = 0; i < 3; ++i) {
    wd[i].resize(w[i].size());
    const uint64_t rows = i < 2 ? I : H, cols = i < 2 ? H : I;
    if (affx_dense_fp8_to_device_layout(w[i].data(), wd[i].data(), rows, cols, nullptr) != 0) return 1;
  }
  affx_shared_expert S{};
  S.gate = {wd[0].data(), sc[0].data(), I, H};
  S.up = {wd[1].data(), sc[1].data(), I, H};
  S.down = {wd[2].data(), sc[2].data(), H, I};
  S.hidden = H;
  S.inter = I;
  S.swiglu_limit = 10.0f;
  bool ok = true;
  // decode: M tokens, accumulated into a y that already holds something (the routed sum); also one
  // token (its own instantiation) and three tokens read dim-major (the strided form)
  for (const uint32_t Md : {1u, 3u, M}) {
    const bool dim_major = Md == 3;
    std::vector<float> x((size_t)Md * H), xt((size_t)Md * H), y0((size_t)Md * H), y, yref;
    for (auto& v : x) v = nd(rng);
    for (auto& v : y0) v = 0.01f * nd(rng);
    for (uint32_t t = 0; t < Md; ++t)
      for (uint32_t h = 0; h < H; ++h) xt[(size_t)h * Md + t] = x[(size_t)t * H + h];
    y = y0;
    yref = y0;
    std::vector<uint8_t> ws(affx_shared_decode_workspace_size(Md, H, I));
    const int rc = dim_major
        ? affx_shared_expert_decode(&S, xt.data(), 1, Md, Md, y.data(), H, 1, 1, ws.data(), ws.size(), nullptr)
        : affx_shared_expert_decode(&S, x.data(), H, 1, Md, y.data(), H, 1, 1, ws.data(), ws.size(), nullptr);
    for (uint32_t t = 0; t < Md; ++t)
      orc_shared_expert(w[0].data(), sc[0].data(), w[1].data(), sc[1].data(), w[2].data(), sc[2].data(), H, I, 10.0f,
                        x.data() + (size_t)t * H, yref.data() + (size_t)t * H);
    // the shared expert's own contribution, compared on its own
    std::vector<float> d(y.size()), dref(y.size());
    for (size_t i = 0; i < y.size(); ++i) { d[i] = y[i] - y0[i]; dref[i] = yref[i] - y0[i]; }
    const double e = rel_l2(d, dref);
    printf("shared decode M=%u%s: rc=%d rel_l2=%.3e\n", Md, dim_major ? " (dim-major)" : "", rc, e);
    ok = ok && rc == 0 && e <= 1e-3;
  }
  // batch: T bf16 tokens, with and without a low part, stored (accumulate 0); the library-GEMM
  // form (bf16 weights, the SwiGLU output as two bf16 terms) and the fp8 MFMA form
  for (int form = 0; form < 4; ++form) {
    const int lo = form & 1, mfma = form >> 1;
    if (mfma)
      setenv("AFFX_SHARED_BATCH", "mfma", 1);
    else
      unsetenv("AFFX_SHARED_BATCH");
    std::vector<float> xf((size_t)T * H), xr((size_t)T * H);
    std::vector<uint16_t> xh((size_t)T * H), xl((size_t)T * H);
    for (size_t i = 0; i < xf.size(); ++i) {
      xf[i] = nd(rng) * (i % 97 == 0 ? 8.0f : 1.0f);
      xh[i] = bf16(xf[i]);
      float hi;
      uint32_t u = (uint32_t)xh[i] << 16;
      memcpy(&hi, &u, 4);
      xl[i] = bf16(xf[i] - hi);
      float lw;
      u = (uint32_t)xl[i] << 16;
      memcpy(&lw, &u, 4);
      xr[i] = lo ? hi + lw : hi;
    }
    std::vector<float> y((size_t)T * H, 123.0f), yref((size_t)T * H, 0.f);
    std::vector<uint8_t> ws(affx_shared_batch_workspace_size(T, H, I));
    const int rc = affx_shared_expert_batch(&S, xh.data(), lo ? xl.data() : nullptr, T, y.data(), 0, ws.data(),
                                            ws.size(), nullptr);
    for (uint32_t t = 0; t < T; ++t)
      orc_shared_expert(w[0].data(), sc[0].data(), w[1].data(), sc[1].data(), w[2].data(), sc[2].data(), H, I, 10.0f,
                        xr.data() + (size_t)t * H, yref.data() + (size_t)t * H);
    const double e = rel_l2(y, yref);
    printf("shared batch T=%u lo=%d %s: rc=%d rel_l2=%.3e\n", T, lo, mfma ? "mfma" : "lib", rc, e);
    ok = ok && rc == 0 && e <= (mfma ? 1e-3 : 1e-5);
  }
  unsetenv("AFFX_SHARED_BATCH");
  // hyper-connection post: single token (every n_hc), batch, and the no-control adds; bit for bit
  for (uint32_t nh : {1u, 2u, 4u, 8u}) {
    std::vector<float> hc((size_t)nh * H), blk(H), post(nh), comb(nh * nh), out((size_t)nh * H), ref((size_t)nh * H);
    for (auto& v : hc) v = nd(rng);
    for (auto& v : blk) v = nd(rng);
    for (auto& v : post) v = nd(rng);
    for (auto& v : comb) v = nd(rng);
    orc_hc_expand(ref.data(), blk.data(), hc.data(), post.data(), comb.data(), H, nh);
    const int rc = affx_hc_post(out.data(), blk.data(), hc.data(), post.data(), comb.data(), H, nh, 1, nullptr);
    bool same = memcmp(out.data(), ref.data(), out.size() * 4) == 0, zero = true;
    for (float v : blk) zero = zero && v == 0.f;
    printf("hc_post n_hc=%u: rc=%d bit-exact=%d block zeroed=%d\n", nh, rc, (int)same, (int)zero);
    ok = ok && rc == 0 && same && zero;
  }
  {
    const uint32_t nh = 4, nb = 5;
    std::vector<uint16_t> hc((size_t)nh * H * nb), out((size_t)nh * H * nb);
    std::vector<float> blk((size_t)H * nb), post(nh * nb), comb(nh * nh * nb);
    for (auto& v : hc) v = bf16(nd(rng));
    for (auto& v : blk) v = nd(rng);
    for (auto& v : post) v = nd(rng);
    for (auto& v : comb) v = nd(rng);
    const std::vector<float> blk0 = blk;
    const int rc = affx_hc_post_batch(out.data(), blk.data(), hc.data(), post.data(), comb.data(), H, nh, nb, 0, nullptr);
    bool same = true;
    for (uint32_t b = 0; b < nb; ++b) {
      std::vector<float> h((size_t)nh * H), bl(H), p(nh), cm(nh * nh), r((size_t)nh * H);
      for (uint32_t s = 0; s < nh; ++s)
        for (uint32_t d = 0; d < H; ++d) {
          const uint32_t u = (uint32_t)hc[((size_t)s * H + d) * nb + b] << 16;
          memcpy(&h[(size_t)s * H + d], &u, 4);
        }
      for (uint32_t d = 0; d < H; ++d) bl[d] = blk0[(size_t)d * nb + b];
      for (uint32_t s = 0; s < nh; ++s) p[s] = post[(size_t)s * nb + b];
      for (uint32_t s = 0; s < nh * nh; ++s) cm[s] = comb[(size_t)s * nb + b];
      orc_hc_expand(r.data(), bl.data(), h.data(), p.data(), cm.data(), H, nh);
      for (uint32_t s = 0; s < nh; ++s)
        for (uint32_t d = 0; d < H; ++d) same = same && out[((size_t)s * H + d) * nb + b] == orc_f32_to_bf16(r[(size_t)s * H + d]);
    }
    const bool kept = blk == blk0;
    printf("hc_post_batch nb=%u: rc=%d bit-exact=%d block kept=%d\n", nb, rc, (int)same, (int)kept);
    ok = ok && rc == 0 && same && kept;
    // the no-control adds
    std::vector<float> h1(H), r1;
    for (auto& v : h1) v = nd(rng);
    r1 = h1;
    orc_hc_add(r1.data(), blk.data(), H);
    std::vector<float> bcopy(blk.begin(), blk.begin() + H);
    int rc2 = affx_hc_add(h1.data(), bcopy.data(), H, 1, nullptr);
    bool add_ok = rc2 == 0 && memcmp(h1.data(), r1.data(), H * 4) == 0;
    std::vector<uint16_t> hb(hc.begin(), hc.begin() + (size_t)H * nb);
    std::vector<float> bb = blk;
    rc2 = affx_hc_add_batch(hb.data(), bb.data(), (uint64_t)H * nb, 1, nullptr);
    for (size_t i = 0; i < hb.size() && add_ok; ++i) {
      float v;
      const uint32_t u = (uint32_t)hc[i] << 16;
      memcpy(&v, &u, 4);
      add_ok = hb[i] == orc_f32_to_bf16(v + blk[i]) && bb[i] == 0.f;
    }
    printf("hc_add and hc_add_batch: ok=%d\n", (int)(add_ok && rc2 == 0));
    ok = ok && add_ok && rc2 == 0;
    // declined shapes
    const int d1 = affx_hc_post(h1.data(), bcopy.data(), h1.data(), post.data(), comb.data(), H, 3, 0, nullptr);
    affx_shared_expert bad = S;
    bad.swiglu_limit = 0.f;
    std::vector<float> yy(H);
    const int d2 = affx_shared_expert_decode(&bad, h1.data(), H, 1, 1, yy.data(), H, 1, 0, nullptr, 0, nullptr);
    printf("declined: n_hc=3 -> %d, limit 0 -> %d\n", d1, d2);
    ok = ok && d1 == AFFX_DECLINED && d2 != AFFX_OK;
  }
  printf("shared ok=%d\n", (int)ok);
  return ok ? 0 : 1;
}

int run_quant(int argc, char** argv) {
  const uint32_t rows = atoi(argv[2]), cols = atoi(argv[3]);
  std::mt19937_64 rng(atoi(argv[4]));
  std::vector<float> w(rows * cols);
  std::normal_distribution<float> nd;
  for (auto& v : w) v = 0.02f * nd(rng);
  for (uint32_t c = 0; c < 16 && c < cols; ++c) w[c] = 0.f;  // an all-zero block
  const auto cb = load_codebook();
  std::vector<float> cbf(8192);
  orc_unpack_codebook(cb.data(), cbf.data());
  const uint64_t nc = rows * cols * 10 / 32, nf = rows * cols * 6 / 128;
  std::vector<uint8_t> c1(nc), f1(nf), c2(nc), f2(nf);
  std::vector<uint16_t> r1(rows), r2(rows);
  int rc = affx_quantize_matrix(w.data(), rows, cols, cbf.data(), nullptr, c1.data(), f1.data(), r1.data(), nullptr);
  orc_quantize_matrix(w.data(), rows, cols, cbf.data(), nullptr, c2.data(), f2.data(), r2.data());
  const bool ok = c1 == c2 && f1 == f2 && r1 == r2;
  printf("quant rc=%d exact=%d\n", rc, (int)ok);
  return rc == 0 && ok ? 0 : 1;
}

int run_dequant(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]);
  std::mt19937_64 rng(atoi(argv[4]));
  Layer L(hidden, inter, 1, rng);
  bool ok = true;
  for (int m = 0; m < 3; ++m) {
    const uint32_t rows = m < 2 ? inter : hidden, cols = m < 2 ? hidden : inter;
    affx_matrix mat{L.dev.data() + L.off[3 * m], L.dev.data() + L.off[3 * m + 1], L.dev.data() + L.off[3 * m + 2],
                    rows, cols};
    std::vector<float> got(rows * cols), ref(rows * cols);
    if (affx_dequant_matrix(&mat, L.cb.data(), got.data(), nullptr)) return 1;
    orc_dequantize_matrix(L.cont.data() + L.off[3 * m], L.cont.data() + L.off[3 * m + 1],
                          (const uint16_t*)(L.cont.data() + L.off[3 * m + 2]), rows, cols, L.cbf.data(), ref.data());
    ok = ok && memcmp(got.data(), ref.data(), got.size() * 4) == 0;
  }
  printf("dequant exact=%d\n", (int)ok);
  return ok ? 0 : 1;
}

// The failure path of the fused decode's bounded wait, forced from the host: with
// AFFX_DECODE_SPIN_LIMIT=0 every waiting workgroup gives up at once (no poll), sets the error
// bit and runs on; every kernel still exits normally.
int run_timeout(int argc, char** argv) {
  const uint32_t hidden = atoi(argv[2]), inter = atoi(argv[3]), n = atoi(argv[4]), M = atoi(argv[5]),
                 K = atoi(argv[6]);
  std::mt19937_64 rng(atoi(argv[7]));
  Layer L(hidden, inter, n, rng);
  std::vector<float> x(M * hidden), yref(M * hidden, 0.f), w;
  std::vector<uint32_t> sel;
  std::normal_distribution<float> nd;
  for (auto& v : x) v = 0.5f * nd(rng);
  routes(rng, M, K, n, sel, w);
  L.oracle(x.data(), sel.data(), w.data(), M, K, yref.data());
  affx_layer abi = L.abi();
  // the engine's arenas: d_x / d_block f32 [hidden][nb], tokens in columns
  const uint32_t nb = 8;
  std::vector<float> dx((size_t)hidden * nb, 0.f), db((size_t)hidden * nb, 0.f);
  for (uint32_t h = 0; h < hidden; ++h)
    for (uint32_t t = 0; t < M; ++t) dx[(size_t)h * nb + t] = x[(size_t)t * hidden + h];
  const size_t wsb = affx_batch_workspace_size(M, K, n, hidden, inter);
  std::vector<uint8_t> ws(wsb, 0);
  affx_engine_ctx ctx{&abi, 1, dx.data(), db.data(), nb, ws.data(), wsb, nullptr};
  std::vector<uint8_t> handled(M * K, 0);
  // bytes of the sync run that every launch (and every reset) leaves zero: all but the one-pass
  // kernel's epoch and publish flags
  auto sync_nonzero = [&]() {
    uint32_t z = 0;
    for (uint32_t i = 0; i < kSyncRunBytes; ++i) z += ws[i] != 0 && i / 4 != kEpochWord;
    return z;
  };
  // all of it, epoch and publish flags included: zero right after a reset
  auto run_nonzero = [&]() {
    uint32_t z = 0;
    for (uint32_t i = 0; i < kSyncBytes; ++i) z += ws[i] != 0;
    return z;
  };
  bool ok = true;
  // 1. the hook: the wait gives up, the call fails (returns 0, marks nothing), the state is reset
  setenv("AFFX_DECODE_SPIN_LIMIT", "0", 1);
  uint32_t got = affx_expert_ffn_batch(&ctx, 0, sel.data(), w.data(), M, K, handled.data());
  const std::string err = affx_last_error();
  uint32_t marked = 0;
  for (auto h : handled) marked += h;
  printf("hook with spin limit 0: returned %u, marked %u, error \"%s\", sync bytes nonzero after %u\n", got,
         marked, err.c_str(), sync_nonzero());
  ok = ok && got == 0 && marked == 0 && err.find("gave up") != std::string::npos && sync_nonzero() == 0;
  // 2. the direct entry: the launch itself returns OK (nothing is known before the kernel runs);
  // affx_decode_status reports the failure, resets, then reports OK
  std::vector<float> y(M * hidden, 0.f);
  int rc = affx_expert_ffn_decode(&abi, x.data(), hidden, 1, M, sel.data(), w.data(), K, y.data(), hidden, 1, 0,
                                  ws.data(), wsb, nullptr);
  const int st1 = affx_decode_status(ws.data(), 1, nullptr);
  const int st2 = affx_decode_status(ws.data(), 0, nullptr);
  printf("direct with spin limit 0: rc=%d status=%d then %d, sync run nonzero after the reset %u\n", rc, st1, st2,
         run_nonzero());
  ok = ok && rc == 0 && st1 == AFFX_ERR_DEVICE && st2 == AFFX_OK && run_nonzero() == 0;
  // 3. normal waits again: the hook takes every pair and the result is right
  unsetenv("AFFX_DECODE_SPIN_LIMIT");
  std::fill(db.begin(), db.end(), 0.f);
  std::fill(handled.begin(), handled.end(), 0);
  got = affx_expert_ffn_batch(&ctx, 0, sel.data(), w.data(), M, K, handled.data());
  std::vector<float> yd(M * hidden);
  for (uint32_t h = 0; h < hidden; ++h)
    for (uint32_t t = 0; t < M; ++t) yd[(size_t)t * hidden + h] = db[(size_t)h * nb + t];
  const double e = rel_l2(yd, yref);
  printf("hook after reset: returned %u of %u, rel_l2=%.3e, sync bytes nonzero %u, status %d\n", got, M * K, e,
         sync_nonzero(), affx_decode_status(ws.data(), 0, nullptr));
  ok = ok && got == M * K && e <= 1e-3 && sync_nonzero() == 0;
  // 4. the allocation-free entry: a launch that gives up is reported by its own status entry,
  // the reset clears the array's sync run, and the next call is right
  setenv("AFFX_DECODE_SPIN_LIMIT", "0", 1);
  std::vector<float> yn(M * hidden, 0.f);
  rc = affx_expert_ffn_decode_noalloc(&abi, x.data(), hidden, 1, M, sel.data(), w.data(), K, yn.data(), hidden, 1, 0,
                                      nullptr);
  const int na1 = affx_decode_noalloc_status(1, nullptr);
  const int na2 = affx_decode_noalloc_status(0, nullptr);
  unsetenv("AFFX_DECODE_SPIN_LIMIT");
  int rc2 = affx_expert_ffn_decode_noalloc(&abi, x.data(), hidden, 1, M, sel.data(), w.data(), K, yn.data(), hidden,
                                           1, 0, nullptr);
  const int na3 = affx_decode_noalloc_status(0, nullptr);
  const double en = rel_l2(yn, yref);
  printf("noalloc with spin limit 0: rc=%d status=%d then %d; next call rc=%d rel_l2=%.3e status %d\n", rc, na1, na2,
         rc2, en, na3);
  ok = ok && rc == 0 && na1 == AFFX_ERR_DEVICE && na2 == AFFX_OK && rc2 == 0 && en <= 1e-3 && na3 == AFFX_OK;
  printf("timeout path ok=%d\n", (int)ok);
  return ok ? 0 : 1;
}

int run_fit(int argc, char** argv) {
  const uint64_t rows = atoi(argv[2]), cols = atoi(argv[3]), budget = atoi(argv[4]);
  const uint32_t iters = atoi(argv[5]);
  const uint64_t seed = atoi(argv[6]);
  const bool seq = argc > 7 && std::string(argv[7]) == "seq";
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> nd;
  std::vector<float> w(rows * cols);
  for (auto& v : w) v = 0.02f * nd(rng);
  for (uint64_t c = 0; c < cols; ++c) w[3 * cols + c] = 0.0f;             // an all-zero row
  for (uint64_t c = 0; c < 16 && c < cols; ++c) w[c] = 0.0f;               // an all-zero block
  bool ok = true;
  // collection
  const uint64_t bound = affx_collect_samples_bound(rows, cols, budget);
  std::vector<float> got(bound + 16, -1.0f);
  std::vector<uint8_t> cws(affx_collect_samples_workspace_size(rows, cols, budget));
  uint64_t n_got = 0;
  if (affx_collect_samples(w.data(), rows, cols, budget, got.data(), bound, &n_got, cws.data(), cws.size(),
                           nullptr) != 0) return 1;
  const uint64_t n_ref = orc_collect_samples(w.data(), rows, cols, budget, nullptr, 0);
  std::vector<float> ref(n_ref + 1);
  orc_collect_samples(w.data(), rows, cols, budget, ref.data(), n_ref);
  ok = ok && n_got == n_ref && memcmp(got.data(), ref.data(), n_ref * 4) == 0;
  printf("collect: %llu samples, exact=%d\n", (unsigned long long)n_got, (int)ok);
  // the fit
  const size_t wsb = affx_fit_codebook_workspace_size(n_ref);
  std::vector<uint8_t> fws(wsb + 256);
  void* fw = (void*)(((uintptr_t)fws.data() + 255) & ~(uintptr_t)255);
  std::vector<float> cb(kCbFloats + 4, 7.0f), cref(kCbFloats);
  float* cb16 = (float*)(((uintptr_t)cb.data() + 15) & ~(uintptr_t)15);
  std::vector<float> sm(n_ref + 4);
  float* s16 = (float*)(((uintptr_t)sm.data() + 15) & ~(uintptr_t)15);
  memcpy(s16, ref.data(), n_ref * 4);
  if (affx_fit_codebook(s16, n_ref, nullptr, iters, seed, seq ? AFFX_FIT_SEQUENTIAL_PICKS : 0, cb16, fw, wsb,
                        nullptr) != 0) {
    printf("fit failed: %s\n", affx_last_error());
    return 1;
  }
  orc_fit_codebook(ref.data(), n_ref, iters, seed, cref.data());
  uint64_t seq_picks = 0, passes = 0;
  affx_fit_codebook_stats(fw, &seq_picks, &passes, nullptr);
  uint32_t diff = 0;
  for (uint32_t i = 0; i < kCbFloats; ++i) diff += memcmp(&cb16[i], &cref[i], 4) != 0;
  printf("fit: %u of %u floats differ, %llu sequential draws, %llu Lloyd passes\n", diff, kCbFloats,
         (unsigned long long)seq_picks, (unsigned long long)passes);
  ok = ok && diff == 0;
  // projection, packing, unpacking
  if (affx_project_codebook(cb16, kCbFloats, nullptr) != 0) return 1;
  orc_project_codebook(cref.data(), kCbFloats);
  std::vector<uint32_t> pk(kVariants * kLut), pref(kVariants * kLut);
  if (affx_pack_codebook(cb16, pk.data(), nullptr) != 0) return 1;
  orc_pack_codebook(cref.data(), pref.data());
  std::vector<float> un(kCbFloats), uref(kCbFloats);
  if (affx_unpack_codebook(pk.data(), un.data(), nullptr) != 0) return 1;
  orc_unpack_codebook(pref.data(), uref.data());
  const bool pj = memcmp(cb16, cref.data(), kCbFloats * 4) == 0, pkok = pk == pref,
             unok = memcmp(un.data(), uref.data(), kCbFloats * 4) == 0;
  printf("project exact=%d pack exact=%d unpack exact=%d\n", (int)pj, (int)pkok, (int)unok);
  ok = ok && pj && pkok && unok;
  printf("fit ok=%d\n", (int)ok);
  return ok ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  orc_set_threads(4);
  const std::string cmd = argv[1];
  if (cmd == "decode" && argc >= 8) return run_decode(argc, argv);
  if (cmd == "grouped" && argc >= 8) return run_grouped(argc, argv);
  if (cmd == "quant" && argc >= 5) return run_quant(argc, argv);
  if (cmd == "dequant" && argc >= 5) return run_dequant(argc, argv);
  if (cmd == "timeout" && argc >= 8) return run_timeout(argc, argv);
  if (cmd == "slots" && argc >= 8) return run_slots(argc, argv);
  if (cmd == "ffnptr" && argc >= 6) return run_ffnptr(argc, argv);
  if (cmd == "route" && argc >= 6) return run_route(argc, argv);
  if (cmd == "shared" && argc >= 7) return run_shared(argc, argv);
  if (cmd == "fit" && argc >= 7) return run_fit(argc, argv);
  if (cmd == "gemv" && argc >= 6) return run_gemv(argc, argv);
  if (cmd == "steps" && argc >= 5) return run_steps(argc, argv);
  if (cmd == "w8a8" && argc >= 5) return run_w8a8(argc, argv);
  fprintf(stderr, "usage: see header\n");
  return 2;
}
