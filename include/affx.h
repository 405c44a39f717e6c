/*
 * affx.h -- C-ABI of the MI355X (gfx950) routed-expert library, libaffx.so.
 *
 * The library runs the hot path of affinity's routed experts on the 2.875-bpw quad-codebook
 * format (AFF_Q2P875_Q4): fused unpack -> codebook dequantisation -> SwiGLU expert FFN, for
 * batch-1/speculative decode (M <= 8 tokens) and for grouped prefill. Every entry point replaces
 * one of the reference engine's C++ entry points; the comment on each names it (file:line in the
 * reference tree). Plain pointers and sizes only: no C++ or torch types cross this boundary.
 *
 * Conventions
 *  - Device pointers are `const void*` / `void*` and must be device memory of the current HIP
 *    device; host pointers are marked `host`. Streams are `hipStream_t` passed as `void*`
 *    (NULL = the default stream). Every call is stream-ordered and does not synchronise, except
 *    where noted.
 *  - Status: 0 = done, AFFX_DECLINED (>0) = preconditions not met and nothing was launched (the
 *    caller falls back, the reference's `bool` false), negative = error. `affx_last_error()`
 *    returns the message of the calling thread's last non-zero status. The reference aborts on
 *    any HIP failure (AFF_HIP_CHECK, src/gpu/hip_common.h:38-46); the C++ shim in INTEGRATION.md
 *    restores that by aborting on a negative status.
 *  - Expert bytes. A *container expert* is the reference's on-disk expert: nine planes
 *    (gate/up/down x codes/fields/rscales) at the offsets `affx_expert_layout` returns,
 *    stride = 9,060,352 B at hidden 4096 / inter 2048 (src/format/aff_format.cpp:45-91). A
 *    *device expert* has the same stride and the same plane offsets, but inside each code and
 *    field plane the 80-byte code runs and 12-byte field runs of every 256-column row segment
 *    are permuted into wave tiles (16 rows x 1024 columns, one run per lane) so that one
 *    128-bit load per lane per run is coalesced. Row scales are unchanged. The permutation is a
 *    bijection on bytes (`affx_expert_to_device_layout` / `..._from_device_layout`).
 *  - The codebook is the container's `__codebook`: uint32[2 variants x 1024], dword v*1024+c,
 *    byte p = E4M3 (OCP fn) encoding of quad element p, every stored exponent in 1..7.
 *  - Shapes: hidden % 1024 == 0, inter % 1024 == 0 (the V4 shapes 4096 / 2048).
 */
#ifndef AFFX_H
#define AFFX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AFFX_OK 0
#define AFFX_DECLINED 1
#define AFFX_ERR_ARG (-1)
#define AFFX_ERR_HIP (-2)
#define AFFX_ERR_DEVICE (-3)
#define AFFX_ERR_CODEBOOK (-4)

#define AFFX_MAX_DECODE_TOKENS 8 /* M of the multi-row decode path */
#define AFFX_MAX_TOPK 16         /* the reference's plan limit (src/gpu/moe_plan.hip:407-420) */
#define AFFX_MAX_EXPERTS 512

/* One quantised matrix in device layout. Mirrors DeviceMatrix{data,scales,rscales,rows,cols}
 * (src/gpu/expert_kernel_hip.h:133-138); codes/fields are the permuted planes. */
typedef struct affx_matrix {
  const void* codes;   /* device: rows*cols*10/32 bytes, wave-tile order */
  const void* fields;  /* device: rows*cols*6/128 bytes, wave-tile order */
  const void* rscales; /* device: bf16[rows] */
  uint32_t rows, cols;
} affx_matrix;

/* One expert's three matrices, each anywhere in device memory. Mirrors DeviceExpert{gate, up,
 * down} (src/gpu/expert_kernel_hip.h:259-261); affx_matrix has DeviceMatrix's field order, so an
 * array of DeviceExpert can be passed as it is (INTEGRATION.md shows the static checks). */
typedef struct affx_device_expert {
  affx_matrix gate, up, down;
} affx_device_expert;

/* Where a layer's experts live: expert e at base + e*stride (device layout), the O(1)
 * addressing of AffReader::expert_ptr (src/format/aff_reader.h:45-48). */
typedef struct affx_layer {
  const void* base;
  uint64_t stride;
  uint32_t n_experts;
  uint32_t hidden, inter;
  const void* codebook; /* device: uint32[2048] */
  float swiglu_limit;   /* the SwiGLU clamp L of src/engine/model.h:52 (10 for V4-Flash). Must be
                           in (0, 1e6]: the kernels scale the SwiGLU output by 2^(7 - ilogb(L^2)),
                           which needs the clamp's bound. The reference's "no clamp" (L <= 0,
                           src/engine/ops.cpp:47-60) is declined (AFFX_DECLINED, nothing
                           launched), so a caller without a clamp takes its own path. */
} affx_layer;

/* ---- library / device --------------------------------------------------------------------- */

/* Checks that the current device is gfx950 and records its CU count. The reference's
 * hip_available() (src/gpu/expert_kernel_hip.h:410). */
int affx_init(void);
const char* affx_last_error(void);
const char* affx_version(void);

/* ---- format ------------------------------------------------------------------------------- */

/* Plane offsets/sizes of one expert (order gate/up/down x codes/fields/rscales) and the stride.
 * compute_expert_layout (src/format/aff_format.cpp:45-91). Host-only, no device needed. */
uint64_t affx_expert_layout(uint64_t hidden, uint64_t inter, uint64_t off9[9], uint64_t size9[9]);

/* 1 when every byte of the packed codebook has stored exponent 1..7 (so a block scale is an
 * exponent add that cannot reach NaN), else 0. The load-time check of StaticPlacement::init
 * (src/gpu/static_placement.hip:938-951). host pointer. */
int affx_codebook_valid(const uint32_t* codebook_host);

/* Host byte permutation of one expert, container -> device layout and back.
 * expert_transpose_planes_host (src/gpu/expert_kernel.hip:2889-2907, expert_kernel_hip.h:78-84).
 * host pointers, `stride` bytes each, src != dst. */
int affx_expert_to_device_layout(const void* src_host, void* dst_host, uint64_t hidden,
                                 uint64_t inter);
int affx_expert_from_device_layout(const void* src_host, void* dst_host, uint64_t hidden,
                                   uint64_t inter);

/* One matrix's code and field planes, container (row-major bit streams) -> device layout (wave
 * tiles); rows % 16 == 0, cols % 1024 == 0; host pointers, no overlap. Row scales are not
 * permuted. expert_transpose_plane_host (src/gpu/expert_kernel_hip.h:78-80), the per-matrix upload
 * step of aff-gpucheck (tools/aff_gpucheck.cpp:54-74). */
int affx_matrix_to_device_layout(const void* src_codes, const void* src_fields, void* dst_codes,
                                 void* dst_fields, uint32_t rows, uint32_t cols);

/* The same permutation on the GPU for n experts uploaded in container layout (src and dst are
 * device buffers of n*stride bytes, not overlapping). The upload step of StaticPlacement::init
 * (src/gpu/static_placement.hip:1094-1097), moved onto the device. */
int affx_permute_experts(const void* src_container, void* dst_device, uint64_t n_experts,
                         uint64_t hidden, uint64_t inter, void* stream);

/* ---- the codebook producer (what aff-quantize runs before it quantises) ----------------------
 * The quad format only (4-wide codes, 1024 entries, 2 variants, power-of-two block scales). All
 * pointers are device buffers; calls are stream-ordered. Every result equals the reference CPU
 * path's bit for bit. */

/* collect_normalized_samples (src/quant/blockquant.cpp:386-423, declared blockquant.h:149-154)
 * without importance: every stride-th row of the row-major f32 matrix w (stride = max(1,
 * rows*cols / max(1, max_samples))), rows whose max |w| is 0 skipped, then each 16-block whose
 * max |w| is nonzero as blk[i] / bmax, in row and column order. Writes at most `cap` floats of
 * out and the full count to *n_out (device uint64). The count is at most
 * affx_collect_samples_bound(); ws holds affx_collect_samples_workspace_size() bytes. The call
 * site is aff-quantize's sampling loop (tools/aff_quantize.cpp:420-425). */
uint64_t affx_collect_samples_bound(uint64_t rows, uint64_t cols, uint64_t max_samples);
size_t affx_collect_samples_workspace_size(uint64_t rows, uint64_t cols, uint64_t max_samples);
int affx_collect_samples(const float* w, uint64_t rows, uint64_t cols, uint64_t max_samples,
                         float* out, uint64_t cap, uint64_t* n_out, void* ws, size_t ws_bytes,
                         void* stream);

/* fit_codebook (src/quant/blockquant.cpp:252-384, declared blockquant.h:141-144) for the quad
 * format: samples [n_samples] (16-byte aligned) -> cb [2][1024][4] floats (16-byte aligned), the
 * raw fit before projection. weights must be NULL (aff-quantize passes none,
 * tools/aff_quantize.cpp:430; AFFX_DECLINED otherwise). flags: 0, or
 * AFFX_FIT_SEQUENTIAL_PICKS to take every k-means++ draw by the sequential sums (the same result,
 * slower; for tests). ws: affx_fit_codebook_workspace_size(n_samples) bytes, 256-byte aligned;
 * its first bytes hold the fit's counters afterwards (affx_fit_codebook_stats). */
#define AFFX_FIT_SEQUENTIAL_PICKS 1u
size_t affx_fit_codebook_workspace_size(uint64_t n_samples);
int affx_fit_codebook(const float* samples, uint64_t n_samples, const float* weights,
                      uint32_t iters, uint64_t seed, uint32_t flags, float* cb, void* ws,
                      size_t ws_bytes, void* stream);
/* The last fit's k-means++ draws that took the sequential sums and its Lloyd passes (host
 * values; synchronises the stream). No counterpart in the reference. */
int affx_fit_codebook_stats(const void* ws, uint64_t* seq_picks, uint64_t* passes, void* stream);

/* project_codebook_e4m3 (blockquant.cpp:463-466) with pow2 scales, in place on n floats;
 * pack_codebook_e4m3_quads (468-480): cb [2048][4] -> packed [2048] dwords;
 * unpack_codebook_e4m3_quads (482-492): packed -> cb. The call sites: aff_quantize.cpp:434, 519
 * and 391. */
int affx_project_codebook(float* cb, uint64_t n, void* stream);
int affx_pack_codebook(const float* cb, uint32_t* packed, void* stream);
int affx_unpack_codebook(const uint32_t* packed, float* cb, void* stream);

/* ---- the .aff container ------------------------------------------------------------------- */

/* An open .aff file: one read-only mapping of it, checked. Opaque. */
typedef struct affx_container affx_container;

/* Maps and checks a container as the reference's AffReader::open does (src/format/aff_reader.cpp:
 * 56-118: magic "AFFINITY", version 1, file size, every section inside the file, every layer's
 * experts inside the expert pool) and as its expert tier does at load (src/engine/model.cpp:
 * 335-357, src/gpu/static_placement.hip:918-951): every layer's matrices in the quad format
 * (AFF_Q2P875_Q4) with compute_expert_layout's plane geometry, a __codebook tensor of 2048 packed
 * dwords with every stored exponent in 1..7. AFFX_ERR_ARG with the reason otherwise. */
int affx_container_open(const char* path, affx_container** out);
void affx_container_close(affx_container* c);
uint32_t affx_container_layer_count(const affx_container* c);
/* A layer's expert count, hidden and intermediate size and the container's expert stride. */
int affx_container_layer(const affx_container* c, uint32_t layer, uint32_t* n_experts,
                         uint64_t* hidden, uint64_t* inter, uint64_t* stride);
/* Host address of expert (layer, expert) in the mapping: pool + base_off + expert * stride, the
 * O(1) addressing of AffReader::expert_ptr (src/format/aff_reader.h:45-48). NULL if out of range. */
const void* affx_container_expert_ptr(const affx_container* c, uint32_t layer, uint32_t expert);
/* The __codebook tensor's 2048 dwords (host out[2048]): what affx_layer.codebook holds once on
 * the device (src/engine/model.cpp:335-357, tools/aff_quantize.cpp:262-271). */
int affx_container_codebook(const affx_container* c, uint32_t* out);
/* Uploads every expert of a layer into the device layout at dst (n_experts * stride bytes with
 * the library's stride for the layer's shape), through staging (device, the same size): the
 * experts are copied host -> device as they lie in the file, then permuted on the device
 * (affx_permute_experts). The upload step of StaticPlacement::init
 * (src/gpu/static_placement.hip:1000-1100). Stream-ordered. */
int affx_container_upload_layer(const affx_container* c, uint32_t layer, void* staging, void* dst,
                                void* stream);

/* ---- dequantisation (validation path) ------------------------------------------------------ */

/* out[r*cols + c] = the float the reference's dequantize_matrix produces (bit-exact):
 * rscale * 2^s * (+-1) * e[v][code][(p+rh)%4]. src/quant/blockquant.cpp:793-833; on the GPU the
 * reference checks the same identity through its decode (src/gpu/expert_kernel.hip:594-619). */
int affx_dequant_matrix(const affx_matrix* m, const void* codebook, float* out, void* stream);

/* ---- single-matrix GEMV (the inner API aff-gpucheck binds) ---------------------------------- */

/* y[r] += sum_i weights[i] * (W_i . x)[r] for n_mats matrices of one shape [rows x cols] given as
 * a host array of affx_matrix (planes in device layout): expert_gemv_batch_hip with its arguments
 * unchanged (src/gpu/expert_kernel_hip.h:152-153, expert_kernel.hip:2687-2722), the call of
 * aff-gpucheck's GEMV bandwidth figure (tools/aff_gpucheck.cpp:544-548). weights: device
 * f32[n_mats]; x: device f32[cols], 16-byte aligned; y: device f32[rows], accumulated; codebook:
 * device uint32[2048] (the packed quads the reference passes through a float pointer). Launches
 * of at most 32 matrices (the reference's kMaxBatch), each after the one before; every y element
 * is summed in a fixed order. rows % 16 == 0, cols a multiple of 1024 up to 8192 (AFFX_DECLINED
 * otherwise: the reference needs cols % 512 == 0). The activation enters the MFMA as three E4M3
 * terms per element (relative error below 2^-12 per element); fp32 accumulation. Stream-ordered,
 * no synchronisation. */
int affx_expert_gemv_batch(const affx_matrix* mats, const float* weights, uint32_t n_mats,
                           const void* codebook, const float* x, float* y, void* stream);

/* y[r] += w * (W . x)[r] for one matrix, w a host scalar: expert_gemv_hip with its arguments
 * unchanged (src/gpu/expert_kernel_hip.h:147-148, expert_kernel.hip:2810-2819), the per-matrix
 * check of aff-gpucheck (tools/aff_gpucheck.cpp:278). As the reference's, it synchronises the
 * stream before returning (y is ready); unlike it, it allocates nothing (w travels in the kernel
 * arguments instead of a device singleton). */
int affx_expert_gemv(const affx_matrix* m, const void* codebook, const float* x, float w, float* y,
                     void* stream);

/* ---- decode: M <= 8 tokens, fused gate/up -> SwiGLU -> down -> weighted combine ------------- */

/* Workspace bytes affx_expert_ffn_decode needs for m tokens with top-k routing. The workspace
 * must be zero-filled before its first use: its first 41,216 bytes hold the fused decode's
 * cross-workgroup state: a 256-byte header (the publish counter of the M > 1 kernels, the error
 * word, the batch-1 kernel's launch epoch), one 128-byte release flag per waiting workgroup, and
 * eight copies of one publish-flag dword per workgroup for the batch-1 kernel. Counter and release
 * flags are zero again after every launch; epoch and publish flags only advance. So no call needs
 * a memset, and the calls are safe under graph capture. Word 2 (bytes 8..11) becomes nonzero if a
 * launch ever gave up waiting for the other workgroups (its output is then invalid); it is sticky
 * until affx_decode_status resets the sync run. */
size_t affx_decode_workspace_size(uint32_t m_tokens, uint32_t top_k, uint32_t hidden,
                                  uint32_t inter);

/* Status of a decode workspace: AFFX_OK, or AFFX_ERR_DEVICE when a launch of
 * affx_expert_ffn_decode on it gave up waiting for its workgroups (error word 2 nonzero; that
 * launch's output was invalid). Copies 4 bytes to the host and synchronises `stream`. reset = 1
 * also zeroes the workspace's sync run (counter, error bits, release and publish flags, epoch),
 * which a timed-out launch can leave raised. The counterpart of the reference's periodic device-status read that
 * aborts the process on a bad dispatch (src/gpu/static_placement.hip:1939-1961); the engine hook
 * affx_expert_ffn_batch makes this check itself after every decode call. */
int affx_decode_status(void* workspace, int reset, void* stream);

/* y[t] (+)= sum_j w[t][j] * FFN_{sel[t][j]}(x[t]) for t < m_tokens (<= 8), j < top_k.
 *  x: device f32, element (t, h) at x[t*x_tok_stride + h*x_dim_stride]; y likewise with
 *  y_tok_stride/y_dim_stride. The engine's dim-major arenas d_x/d_block f32 [H][nb_stride]
 *  are tok_stride 1, dim_stride nb_stride. `accumulate` = 1 adds into y (the engine's d_block),
 *  0 overwrites.
 *  sel: device uint32 [m_tokens][top_k]; ids >= n_experts are padding and are skipped (as the
 *  reference's plan does, src/gpu/moe_plan.h:146). w: device f32 [m_tokens][top_k].
 * Replaces the batch-1 GPU FFN expert_ffn_hip (src/gpu/expert_kernel.hip:2737-2808,
 * expert_kernel_hip.h:273) and the narrow NT=1 arm of the W8A8 GEMM that the engine's decode uses
 * (expert_kernel.hip:3049-3058). One persistent launch (routing plan, activation split, gate/up +
 * SwiGLU, down + combine; between gate/up and down, an agent-scope publish counter whose last
 * adder raises one release flag per down-phase workgroup, or at batch 1 one publish flag per
 * workgroup that the down-phase workgroups poll); it needs every
 * workgroup of its grid resident at once, so the grid is sized to the device, and it falls back to
 * the staged launches below when the device cannot hold it. No host synchronisation. */
int affx_expert_ffn_decode(const affx_layer* layer, const float* x, uint64_t x_tok_stride,
                           uint64_t x_dim_stride, uint32_t m_tokens, const uint32_t* sel,
                           const float* w, uint32_t top_k, float* y, uint64_t y_tok_stride,
                           uint64_t y_dim_stride, int accumulate, void* workspace,
                           size_t workspace_bytes, void* stream);

/* affx_expert_ffn_decode for callers that cannot allocate: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. No counterpart in the reference (its decode
 * takes caller-owned scratch). Same arguments without the workspace: the library keeps it in a
 * static device array of 3.25 MiB per GPU (held until the process ends), set up by affx_init (or
 * by the first call on a device) and shared by every call on that GPU, so calls that overlap on
 * one GPU (other streams, other threads) race. Serves m_tokens <= 8, m_tokens * top_k <= 64,
 * hidden <= 4096, inter <= 2048; larger sizes return AFFX_ERR_ARG with a message. Calls no
 * hipMalloc, hipFree or allocating routine. The set-up zeroes the array and synchronises once;
 * a first call on a device made under graph capture (which cannot synchronise) is refused with a
 * message: call affx_init on that device before capturing. A launch whose workgroups gave up
 * waiting for each other is reported by affx_decode_noalloc_status, as the workspace entry's by
 * affx_decode_status. */
int affx_expert_ffn_decode_noalloc(const affx_layer* layer, const float* x, uint64_t x_tok_stride,
                                   uint64_t x_dim_stride, uint32_t m_tokens, const uint32_t* sel,
                                   const float* w, uint32_t top_k, float* y, uint64_t y_tok_stride,
                                   uint64_t y_dim_stride, int accumulate, void* stream);

/* affx_decode_status for the current device's allocation-free decode array (no counterpart in the
 * reference; for the callers affx_expert_ffn_decode_noalloc serves): AFFX_OK, or AFFX_ERR_DEVICE
 * when a launch on the array gave up waiting for its workgroups (its output was invalid); reset = 1
 * then zeroes the array's sync run (with a fill kernel on `stream`) so the next call is right.
 * Copies 4 bytes to the host and synchronises `stream`. */
int affx_decode_noalloc_status(int reset, void* stream);

/* out[h] += sum_k weights[k] * FFN_k(x)[h] for one token through n_experts experts given as a
 * host array of per-matrix device pointers (planes in device layout): expert_ffn_hip with its
 * arguments unchanged (src/gpu/expert_kernel_hip.h:273, expert_kernel.hip:2737-2808), the call
 * aff-gpucheck makes (tools/aff_gpucheck.cpp:498, 585). weights: device f32[n_experts]; x: device
 * f32[hidden]; out: device f32[hidden], accumulated; codebook: device uint32[2048] (the packed
 * quads the reference passes through a float pointer). scratch: device, the reference's
 * 2 * n_experts * inter floats, no clearing needed (it holds the plan and the SwiGLU terms; each
 * gate/up workgroup makes the activation terms in its own LDS), for any n_experts from 1 to 16
 * (the reference's 32 matrices per launch); shapes as the layer entries. Three stream-ordered
 * launches (the staged decode: routing plan, gate/up + SwiGLU, down + combine), no
 * synchronisation. AFFX_DECLINED when a shape or the count is outside this. */
int affx_expert_ffn(const affx_device_expert* experts, const float* weights, uint32_t n_experts,
                    const void* codebook, const float* x, float swiglu_limit, float* scratch,
                    float* out, void* stream);

/* The same three steps as separate stream-ordered calls (same workspace, same arguments), for
 * callers that interleave other work or time the stages, as the reference's GPU FFN is three
 * launches: activation prep + routing plan (batch_quant_fp8_hip, src/gpu/batch_kernels.h:124;
 * moe_plan_hip, src/gpu/moe_plan.hip:407-420), gate/up + SwiGLU (expert_gemv_split_hip +
 * swiglu_all_kernel, src/gpu/expert_kernel.hip:2616-2662, 114-129) and down + combine
 * (expert_gemv_multix_hip, src/gpu/expert_kernel.hip:2573-2609). */
int affx_decode_prepare(const affx_layer* layer, const float* x, uint64_t x_tok_stride,
                        uint64_t x_dim_stride, uint32_t m_tokens, const uint32_t* sel,
                        const float* w, uint32_t top_k, void* workspace, size_t workspace_bytes,
                        void* stream);
int affx_decode_gateup(const affx_layer* layer, uint32_t m_tokens, uint32_t top_k,
                       void* workspace, size_t workspace_bytes, void* stream);
int affx_decode_down(const affx_layer* layer, uint32_t m_tokens, uint32_t top_k, float* y,
                     uint64_t y_tok_stride, uint64_t y_dim_stride, int accumulate,
                     void* workspace, size_t workspace_bytes, void* stream);

/* affx_expert_ffn_decode as the three staged launches above, in one call (same arguments; no
 * counterpart of its own in the reference: it is the staged form of the same decode, for
 * comparison and for devices that cannot hold the persistent grid). */
int affx_decode_staged(const affx_layer* layer, const float* x, uint64_t x_tok_stride,
                       uint64_t x_dim_stride, uint32_t m_tokens, const uint32_t* sel,
                       const float* w, uint32_t top_k, float* y, uint64_t y_tok_stride,
                       uint64_t y_dim_stride, int accumulate, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---- prefill: grouped GEMM over an expert-sorted slot list ---------------------------------- */

/* Workspace bytes of affx_moe_plan + affx_expert_ffn_grouped for n_tok tokens, top-k routing. */
size_t affx_grouped_workspace_size(uint32_t n_tok, uint32_t top_k, uint32_t n_experts,
                                   uint32_t hidden, uint32_t inter);

/* y[t] (+)= sum_j w[t][j] * FFN_{sel[t][j]}(x[t]) for all n_tok tokens, grouped by expert:
 * every expert's weights are decoded once per tile of its tokens (96 tokens for gate/up with a
 * bf16 x, 60 otherwise) and reused for all of the tile's tokens.
 *  x: device bf16 [n_tok][hidden] (token-major); x_lo: optional second bf16 term (x = x + x_lo)
 *  for f32 activations split hi/lo, or NULL. Both 16-byte aligned (else AFFX_ERR_ARG).
 *  sel/w: device [n_tok][top_k]; padding ids >= n_experts skipped.
 *  y: device f32 [n_tok][hidden] (token-major).
 * Replaces run_batch_device's prefill sequence (src/gpu/static_placement.hip:1348-1964):
 * moe_plan_hip (src/gpu/moe_plan.hip:407-420) -> batch_quant_fp8_hip -> expert_gemm_wmma_hip
 * gate/up (expert_kernel.hip:3018-3062) -> expert_swiglu_quant_hip -> expert_gemm_wmma_hip down
 * -> expert_scatter_slots_hip (expert_kernel.hip:935-947). Deterministic: every output element
 * is summed in a fixed order, no float atomics. */
int affx_expert_ffn_grouped(const affx_layer* layer, const void* x, const void* x_lo,
                            uint32_t n_tok, const uint32_t* sel, const float* w, uint32_t top_k,
                            float* y, int accumulate, void* workspace, size_t workspace_bytes,
                            void* stream);

/* The same prefill over a slot list the caller has already built on the device, the shape of the
 * reference engine's device plan (MoePlanArgs, src/gpu/moe_plan.h:144-170, from moe_plan_kernel,
 * src/gpu/moe_plan.hip:116-380): slots sorted by expert, expert e owning slots
 * [expert_start[e], expert_start[e+1]) (n_experts + 1 entries); tok[s] the token of slot s and
 * wt[s] its router weight; ord the slots sorted by token, token t's being
 * ord[run[t] .. run[t+1]) (run: n_tok + 1 entries). Token t's output sums its slots in ord order.
 * x, x_lo, y as affx_expert_ffn_grouped; all arrays device memory. Workspace:
 * affx_grouped_workspace_size(n_tok, top_k, ...) for any top_k with n_tok * top_k >= n_slots.
 * The entry trusts the list's consistency but not its bounds: indices are clamped on the device
 * (a bad list gives wrong output, never an access outside the buffers). affx_expert_ffn_grouped
 * is this entry after building the list from the routes on the device, a token's slots in route
 * order. */
int affx_expert_ffn_grouped_slots(const affx_layer* layer, const void* x, const void* x_lo,
                                  uint32_t n_tok, const uint32_t* expert_start, const uint32_t* tok,
                                  const float* wt, const uint32_t* ord, const uint32_t* run,
                                  uint32_t n_slots, float* y, int accumulate, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* ---- the reference's separable batch-pipeline steps ------------------------------------------
 * For a caller that drives the reference's own step sequence (run_batch_device's prefill arm:
 * gather -> W8A8 GEMM -> SwiGLU + requantise -> W8A8 GEMM -> fixed-order scatter,
 * src/gpu/static_placement.hip:1856-1914). affx_expert_ffn_grouped(_slots) fuses these into its
 * grouped GEMM and combine; these keep the reference's formats. Device pointers, stream-ordered,
 * no synchronisation. */

/* SwiGLU times the router weight, then the E4M3 requantise: expert_swiglu_quant_hip with its
 * arguments unchanged (src/gpu/expert_kernel_hip.h:238-240, expert_kernel.hip:862-931, 2822-2835).
 * g, u: bf16 [dim][total] (dim-major, one column per slot); w: f32 [total] or NULL (weight 1);
 * v = silu(min(g, L)) * clamp(u, -L, L) * w (no clamp when limit <= 0). Per (slot, 128-row band):
 * scales[slot][band] = max |v| / 448 (1 when the band is zero), out[slot][k] (E4M3, slot-major
 * [total][dim]) = E4M3(clamp(v / scale, +-448)), round to nearest even. dim % 128 == 0, out
 * 16-byte aligned (AFFX_ERR_ARG otherwise). */
int affx_expert_swiglu_quant(const uint16_t* g, const uint16_t* u, const float* w, uint8_t* out,
                             float* scales, uint32_t dim, uint32_t total, float limit, void* stream);

/* Fixed-order reduction of a [dim][total] bf16 slot arena into the chunk's f32 accumulator:
 * expert_scatter_slots_hip with its arguments unchanged (src/gpu/expert_kernel_hip.h:249-251,
 * expert_kernel.hip:935-947, 2837-2843). block[h * nb_stride + t] += sum over i in
 * run[t] .. run[t+1]-1, in that order from zero, of y[h * total + ord[i]]; tokens whose run is
 * empty are not written. Every ord[i] < total (not checked, as in the reference). Deterministic (no
 * atomics). dim <= 65535. */
int affx_expert_scatter_slots(const uint16_t* y, float* block, const uint32_t* ord, const uint32_t* run,
                              uint32_t dim, uint32_t nb_tok, uint32_t nb_stride, uint32_t total,
                              void* stream);

/* nt token columns of a dim-major [dim][nb] arena into a compact [dim][nt] tile:
 * dst[c * nt + t] = src[c * nb + tok[t]], every tok[t] < nb (not checked, as in the reference).
 * expert_gather_tokens_hip with its arguments unchanged (src/gpu/expert_kernel_hip.h:255-256,
 * expert_kernel.hip:828-835, 1673-1680). */
int affx_expert_gather_tokens(const float* src, float* dst, const uint32_t* tok, uint32_t dim,
                              uint32_t nb, uint32_t nt, void* stream);

/* One expert matrix's share of a W8A8 GEMM launch. Mirrors ExpertTile (src/gpu/expert_kernel_hip.h:
 * 200-215) field for field: codes/fields/rscales are one matrix's planes in device layout (as in
 * affx_matrix), tok = nt token ids into the activation's rows (NULL: 0 .. nt-1), y = the output
 * [rows][ld] (ld = 0: a compact [rows][nt] block), f32 or bf16 by the launch's y_bf16. */
typedef struct affx_expert_tile {
  const void* codes;
  const void* fields;
  const void* rscales;
  const uint32_t* tok;
  void* y;
  uint32_t nt;
  uint32_t ld;
} affx_expert_tile;

/* The single-matrix W8A8 GEMM between the steps above: expert_gemm_wmma_hip with its arguments
 * (src/gpu/expert_kernel_hip.h:217-228; kernel expert_kernel.hip:364-825, host 3018-3062). tiles:
 * a DEVICE array of n_tiles descriptors (nt = 0 is a pad and writes nothing), every nt <= max_nt <=
 * 64. x8: E4M3 activations token-major [tokens][cols]; xs: f32 [tokens][cols / 128], one scale per
 * (token, 128-column block); codebook: the packed uint32[2048] (the reference passes the same bytes
 * as `const float* cb`). For each tile, row r < rows and column j < nt, t = tok ? tok[j] : j:
 *   out = sum over blocks kb in order of fmaf(raw_kb, xs[t][kb], out), raw_kb = sum over the
 *         block's 128 columns of W8[r][k] * x8[t][k] (W8: the weight's E4M3 value without the row
 *         scale: codebook entry, block exponent add, sign, rotation);
 *   y[r * (ld ? ld : nt) + j] = out * (bf16 rscales[r] * wscale), stored f32, or bf16 rounded to
 *         nearest even when y_bf16.
 * rows % 16 == 0, cols % 1024 == 0 (AFFX_DECLINED otherwise, as for max_nt > 64); x8 and xs
 * 16-byte aligned. Stream-ordered, no synchronisation. */
int affx_expert_gemm_w8a8(const affx_expert_tile* tiles, uint32_t n_tiles, uint32_t max_nt, const void* x8,
                          const float* xs, const uint32_t* codebook, uint32_t rows, uint32_t cols, float wscale,
                          int y_bf16, void* stream);

/* ---- routing on the device ------------------------------------------------------------------ */

#define AFFX_ROUTE_ENGINE 0  /* the engine router: sqrtsoftplus scores, bias for selection only */
#define AFFX_ROUTE_SOFTMAX 1 /* the benchmark configs: top-k logits, softmax over the k */

/* Top-k routing of n_tok tokens from their router logits, on the device, writing the
 * sel/w [n_tok][top_k] (token-major, device) that affx_expert_ffn_decode and
 * affx_expert_ffn_grouped read, so routes never pass through the host. Logit (t, e) at
 * logits[t * tok_stride + e * expert_stride]: token-major [n_tok][n_expert] is (n_expert, 1), the
 * engine's dim-major batch arena [n_expert][nb] is (1, nb).
 * AFFX_ROUTE_ENGINE: route_topk (src/engine/ops.cpp:62-92; the device form router_topk_kernel,
 * src/gpu/batch_kernels.hip:2964-3031, called from the layer loop at src/engine/model.cpp:
 * 1582-1599): score = sqrt(softplus(logit)) (x > 20 taken as is), the top_k largest of
 * score + bias[e] (bias: device f32[n_expert] or NULL), ties to the lower id; weight = score *
 * inv * routed_scaling, inv = 1 / max(sum of the k scores in double, 2^-14) if norm_topk_prob,
 * else 1. The scores are within an ulp of the host's float libm (so the weights within a few).
 * AFFX_ROUTE_SOFTMAX: the top_k largest logits (ties to the lower id), weights the softmax over
 * those k in double (bias, norm_topk_prob and routed_scaling unused).
 * top_k <= min(16, n_expert), n_expert <= 512. One wave per token; no synchronisation. */
int affx_route_topk(const float* logits, uint64_t tok_stride, uint64_t expert_stride,
                    const float* bias, uint32_t n_tok, uint32_t n_expert, uint32_t top_k, int rule,
                    int norm_topk_prob, float routed_scaling, uint32_t* sel, float* w, void* stream);

/* ---- the step after: shared expert and hyper-connection post -------------------------------- */

/* One FP8 dense matrix: the reference's DenseW with quant AFF_FP8_E4M3 (src/engine/ops.h:142-151;
 * format src/engine/matvec_fp8.inc:8-10). data: device E4M3 bytes of the [rows x cols] matrix in
 * the device layout affx_dense_fp8_to_device_layout writes (the container's row-major bytes,
 * permuted once at upload), 16-byte aligned; scales: device UE8M0 bytes, one per 128 x 128 tile,
 * row-major [rows / 128][cols / 128] as the container holds them, 4-byte aligned. E4M3 0x7F / 0xFF
 * are NaN (as in the reference's scalar decode, src/quant/source_dtypes.cpp:24-25). */
typedef struct affx_dense_fp8 {
  const void* data;
  const uint8_t* scales;
  uint64_t rows, cols;
} affx_dense_fp8;

/* The shared expert of a layer: gate, up [inter x hidden] and down [hidden x inter] (the
 * reference's shexp_gate/up/down, src/engine/model.h:125-127), hidden and inter multiples of 1024
 * (inter <= 8192; hidden <= 4096 for decode, 8192 for the batch), the SwiGLU clamp limit in
 * (0, 1e6] (see affx_layer). */
typedef struct affx_shared_expert {
  affx_dense_fp8 gate, up, down;
  uint32_t hidden, inter;
  float swiglu_limit;
} affx_shared_expert;

/* The container's row-major E4M3 bytes (device, src) into the device layout (device, dst, a
 * different buffer) the shared-expert kernels read: 2 KiB per (16-row tile, 128-column step),
 * [half][lane][16 B], lane c + 16 kg holding row 16 tile + c, columns 128 step + 64 half + 16 kg
 * .. + 15: the scaled fp8 MFMA's fragment order. rows % 16 == 0, cols % 128 == 0. The
 * counterpart of the reference's preshuffle of these same tensors into its WMMA fragment order
 * at registration (preshuffle_fp8_hip, src/gpu/dense_gpu.hip:940-965; the allowlist ps_for,
 * 791-813, names shexp_gate/up/down). Stream-ordered. */
int affx_dense_fp8_to_device_layout(const void* src, void* dst, uint64_t rows, uint64_t cols, void* stream);

size_t affx_shared_decode_workspace_size(uint32_t m_tokens, uint32_t hidden, uint32_t inter);
/* The batch's workspace: 8 * inter * hidden bytes of widened weights plus 12 * inter bytes a token
 * (n_tok = 4096, hidden 4096, inter 2048: 160 MiB). */
size_t affx_shared_batch_workspace_size(uint32_t n_tok, uint32_t hidden, uint32_t inter);

/* The shared expert on m_tokens <= 8 tokens: y[t] (+)= W_d . swiglu(W_g x[t], W_u x[t]).
 * Replaces DenseOps::shexp (src/engine/model.h:314-319; DenseGpu::shexp, src/gpu/dense_gpu.hip:
 * 2030-2116) for a resident shared expert: accumulate = 1 is its out == nullptr form (added into
 * the device block the routed experts wrote), 0 stores. x and y as in affx_expert_ffn_decode
 * (element (t, h) at x[t * x_tok_stride + h * x_dim_stride]). The host composition it matches is
 * src/engine/model.cpp:1214-1222. Accumulating after the routed experts on the same stream gives
 * the host's order: block = routed sum, then block += shared. Two launches (gate/up + SwiGLU,
 * down), no synchronisation. */
int affx_shared_expert_decode(const affx_shared_expert* shexp, const float* x, uint64_t x_tok_stride,
                              uint64_t x_dim_stride, uint32_t m_tokens, float* y, uint64_t y_tok_stride,
                              uint64_t y_dim_stride, int accumulate, void* workspace, size_t workspace_bytes,
                              void* stream);

/* The shared expert on a chunk of n_tok tokens: y[t] (+)= W_d . swiglu(W_g x[t], W_u x[t]) for
 * every token. Replaces BatchOps::shexp (src/engine/model.h:504-505; DenseGpu::batch_shexp,
 * src/gpu/dense_gpu.hip:4897-4950, which accumulates into the batch block). x (and x_lo, or NULL)
 * bf16 [n_tok][hidden] as in affx_expert_ffn_grouped (x_lo carries the low part of an f32
 * input); y f32 [n_tok][hidden]; these and the workspace 16-byte aligned. accumulate = 0 stores
 * without reading y.
 * The weights are widened to bf16 in the workspace (exact) and the two GEMMs run in hipBLASLt with
 * f32 accumulation, the SwiGLU output between them as two bf16 terms (about 16 significant
 * bits); a shape the library has no algorithm for, or the environment variable
 * AFFX_SHARED_BATCH=mfma, takes the library's own fp8 MFMA kernels instead (activations as E4M3
 * terms, about 3e-4 relative L2 on random codes). Four launches (five with x_lo), no
 * synchronisation; the first call for a token count asks hipBLASLt's heuristic on the host, so it
 * must not be the one a graph capture records. */
int affx_shared_expert_batch(const affx_shared_expert* shexp, const void* x, const void* x_lo, uint32_t n_tok,
                             float* y, int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/* The sublayer's hyper-connection post for one token, with a control: lane dst of out_hc
 * [n_hc][n_embd] = block * post[dst] + sum over src in order of comb[dst + src * n_hc] * hc lane
 * src, bit for bit the host's hc_expand (src/engine/ops.cpp:470-482). Replaces DenseGpu::hc_post's
 * control arm (src/gpu/dense_gpu.hip:2394-2465, hc_expand_reg_kernel 1703-1710). zero_block = 1
 * leaves the block zero for the next sublayer, as the reference's kernel does. n_hc in {1, 2, 4,
 * 8} (the reference silently runs 4 for any other value; this declines it). All f32, device. On
 * one GPU the block is already whole: the sublayer's block_reduce (model.cpp:1759-1762) is the
 * identity and there is no exchange to fold in. */
int affx_hc_post(float* out_hc, float* block, const float* hc, const float* post, const float* comb,
                 uint32_t n_embd, uint32_t n_hc, int zero_block, void* stream);

/* hc_post for a layer without a control: lane 0 += block (src/engine/model.cpp:1237-1238;
 * hc_add_kernel, src/gpu/dense_gpu.hip:1717-1724). */
int affx_hc_add(float* hc, float* block, uint32_t n_embd, int zero_block, void* stream);

/* The batch form over the engine's dim-major arenas of nb tokens (batch_hc_post,
 * src/gpu/dense_gpu.hip:4517-4534; batch_hc_expand_reg_kernel, src/gpu/batch_kernels.hip:
 * 1977-2002): hc and out_hc bf16 [n_hc][n_embd][nb], block f32 [n_embd][nb], post f32 [n_hc][nb],
 * comb f32 [n_hc * n_hc][nb]; each result rounded to bf16 (nearest even) once. */
int affx_hc_post_batch(uint16_t* out_hc, float* block, const uint16_t* hc, const float* post, const float* comb,
                       uint32_t n_embd, uint32_t n_hc, uint32_t nb, int zero_block, void* stream);

/* Lane 0 of the bf16 batch state += block over n = n_embd * nb elements, rounded to bf16
 * (batch_hc_add_bf16_kernel, src/gpu/batch_kernels.hip:2011-2018). */
int affx_hc_add_batch(uint16_t* hc, float* block, uint64_t n, int zero_block, void* stream);

/* ---- engine hook ---------------------------------------------------------------------------- */

/* State behind affx_expert_ffn_batch: the per-layer expert tables and the engine's device
 * arenas, as the reference's lambda captures them (tools/affinity.cpp:1218-1235). */
typedef struct affx_engine_ctx {
  const affx_layer* layers; /* [n_layers] */
  uint32_t n_layers;
  const float* d_x;         /* f32 [hidden][nb_stride], dim-major (the engine's d_x) */
  float* d_block;           /* f32 [hidden][nb_stride], accumulated into */
  uint32_t nb_stride;
  void* workspace;          /* device, zero-filled before first use (its first bytes hold the
                               decode's persistent counter and flags; no call disturbs them) */
  size_t workspace_bytes;
  void* stream;
} affx_engine_ctx;

/* ExpertFfnBatch-shaped hook (src/engine/model.h:664-666): takes every (token, expert) pair of
 * host arrays sel/w [nb_tok][k], runs them on the GPU into ctx->d_block, sets handled[b*k+j]=1
 * for each pair taken, returns the count. Padding ids >= n_experts are neither taken nor marked.
 * nb_tok <= 8 runs the decode path, larger batches the grouped path. Returns 0 (nothing taken)
 * on any error, a decode whose workgroups gave up waiting for each other included (the hook
 * then resets the workspace's sync run); affx_last_error() says why. Synchronises the stream
 * before returning (the routes arrive in host memory). */
uint32_t affx_expert_ffn_batch(void* ctx, uint32_t layer, const uint32_t* sel, const float* w,
                               uint32_t nb_tok, uint32_t k, uint8_t* handled);

/* Workspace bytes affx_expert_ffn_batch needs for a batch of nb_tok tokens (the reference sizes
 * its per-rank arenas the same way, growing them on demand: grow_w8a8,
 * src/gpu/static_placement.hip:1254-1346). */
size_t affx_batch_workspace_size(uint32_t nb_tok, uint32_t top_k, uint32_t n_experts,
                                 uint32_t hidden, uint32_t inter);

/* ---- producer: synthetic weights and the codebook quantiser on the GPU ---------------------- */

/* out[i] = bf16_RNE((float)(scale * N_i)) (or the plain float when bf16_round == 0), with N_i
 * the i-th Box-Muller normal of a splitmix64 stream seeded `seed`, two draws per normal: the
 * generator of src/quant/blockquant.cpp:37-42, 862-869 in counter form. out: device f32[n]. */
int affx_gen_normal(uint64_t seed, uint64_t n, double scale, void* out, int bf16_round,
                    void* stream);

/* quantize_matrix (src/quant/blockquant.cpp:586-791) for the quad format on the GPU, bit-exact:
 * w f32 [rows][cols] (cols % 64 == 0, <= 8192) -> codes/fields/rscales in the container's
 * row-major streams. codebook_f32: float[2][1024][4] (the projected E4M3 values). importance:
 * optional f32[cols] column importance, or NULL. All device pointers. */
int affx_quantize_matrix(const void* w, uint32_t rows, uint32_t cols, const void* codebook_f32,
                         const void* importance, void* codes, void* fields, void* rscales,
                         void* stream);

/* One synthetic expert in container layout: gate/up/down = bf16(0.02 N(0,1)) from seeds
 * seed+0/1/2, quantised against codebook_f32. scratch: device f32[inter*hidden]. The quantiser
 * loop of tools/aff_quantize.cpp:589-616 for one expert, with synthetic weights. */
int affx_fill_expert(void* expert, uint64_t hidden, uint64_t inter, const void* codebook_f32,
                     uint32_t seed, void* scratch, void* stream);

/* ---- diagnostics ---------------------------------------------------------------------------- */

/* Runs one v_mfma_scale_f32_16x16x128_f8f6f4 (E4M3 x E4M3, unit scales) on a[64][32] and
 * b[64][32] fp8 bytes (one row per lane) and writes the 64x4 f32 accumulator lanes to d.
 * Device pointers. Lets a test pin the lane layout and the OCP E4M3 interpretation the decode
 * kernels rely on. No reference counterpart (the reference's WMMA layout test, test_wmma, is
 * absent from its tree: CMakeLists.txt:304). */
int affx_selftest_mfma_fp8(const void* a, const void* b, float* d, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* AFFX_H */
