/*
 * fuel_rocm.h -- C ABI of the MI355X (gfx950) quantized-matmul backend for
 * fuel.  Plain pointers and sizes only; device pointers are HIP device
 * addresses on the handle's device.  Every entry point returns a status:
 *
 *   FRQ_OK 0, FRQ_MISALIGNED 1, FRQ_INVALID 2, FRQ_UNSUPPORTED 3,
 *   FRQ_WORKSPACE 4, FRQ_INTERNAL 5
 *
 * the integer convention of fuel's CUDA FFI status codes
 * (fuel-cuda-backend/src/baracuda/status.rs:5-12).  frq_last_error() returns
 * the message of the calling thread's last failure.  Entry points never abort.
 *
 * Two seams of the reference are mirrored:
 *   (1) the trait-object seam QuantizedDeviceKernels + DynQuantizedStorage
 *       (fuel-backend-contract/src/quantized.rs:29-119): frq_qstorage_*;
 *   (2) the lazy-graph KernelRef registered at (OpKind::QMatMul,
 *       [F32, U32, F32], BackendId) (fuel-dispatch/src/dispatch.rs:1638-1718,
 *       5801; fuel-dispatch/src/kernel.rs:168-173, 482-488): frq_qmatmul.
 *
 * Work is enqueued on the device's stream and is asynchronous unless stated;
 * frq_sync waits for it.  Thread safety (the trait seam is Send + Sync,
 * fuel-backend-contract/src/quantized.rs:29): every entry point that enqueues
 * work on a device, or touches its stream or workspace, holds that device
 * handle's lock, so calls from several threads on one handle, or on storages
 * of one handle, take turns on the host and their work runs in call order on
 * the handle's one stream.  A call's results do not depend on which calls
 * came before it in the process (frq_qmatmul_plan reports the kernels a
 * QMatMul runs; they follow from the call alone).
 */
#ifndef FUEL_ROCM_H
#define FUEL_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FRQ_OK = 0,
    FRQ_MISALIGNED = 1,
    FRQ_INVALID = 2,
    FRQ_UNSUPPORTED = 3,
    FRQ_WORKSPACE = 4,
    FRQ_INTERNAL = 5
};

/* GgmlDType codes (fuel-ir/src/quantized.rs:36-76, from_u32 / to_u32). */
enum {
    FRQ_F32 = 0,
    FRQ_F16 = 1,
    FRQ_Q8_0 = 8,
    FRQ_Q4K = 12,
    FRQ_Q6K = 14,
    FRQ_Q8K = 15
};

typedef struct frq_device frq_device;
typedef struct frq_qstorage frq_qstorage;

/* Message of the calling thread's last failed call ("" if none). */
const char *frq_last_error(void);

/* GgmlDType::type_size / block_size (fuel-ir/src/quantized.rs:78-104);
 * 0 for a code this backend does not handle. */
size_t frq_type_size(int ggml_dtype);
size_t frq_block_size(int ggml_dtype);

/* ---- device (the DynBackendDevice handle; fuel-backend-contract/src/dyn_backend.rs:292-398) ---- */
int frq_device_count(int *count);
/* Opens `ordinal` with its own HIP stream. */
int frq_device_open(int ordinal, frq_device **out);
int frq_device_close(frq_device *dev);
/* Use a caller-owned hipStream_t (passed as void*) instead of the device's
 * own stream; NULL restores the device's stream. */
int frq_device_set_stream(frq_device *dev, void *hip_stream);
int frq_sync(frq_device *dev);
int frq_device_cu_count(const frq_device *dev, int *cus);
/* Bytes of device workspace the handle holds (quantized activation rows,
 * split-K partial sums, MoE routing scratch), grown on demand by the calls
 * that need it and released by frq_device_close.  Introspection only. */
int frq_device_workspace_bytes(const frq_device *dev, size_t *bytes);

/* Device memory helpers standing in for DynBackendStorage buffers. */
int frq_malloc(frq_device *dev, size_t bytes, void **dptr);
int frq_free(frq_device *dev, void *dptr);
int frq_memcpy_htod(frq_device *dev, void *dst, const void *src, size_t bytes); /* synchronous */
int frq_memcpy_dtoh(frq_device *dev, void *dst, const void *src, size_t bytes); /* synchronous */
int frq_memcpy_dtod(frq_device *dev, void *dst, const void *src, size_t bytes); /* async */
int frq_memset(frq_device *dev, void *dst, int value, size_t bytes);            /* async */

/* ---- QuantizedDeviceKernels (fuel-backend-contract/src/quantized.rs:108-119) ---- */
/* qzeros(elem_count, dtype): zero blocks; elem_count % block_size == 0. */
int frq_qstorage_zeros(frq_device *dev, int ggml_dtype, size_t elem_count, frq_qstorage **out);
/* load_quantized(dtype, data): copies `nbytes` of block bytes (a multiple of
 * type_size) from host memory to the device, in fuel's block layout. */
int frq_qstorage_load(frq_device *dev, int ggml_dtype, const void *host_bytes, size_t nbytes,
                      frq_qstorage **out);
int frq_qstorage_free(frq_qstorage *qs);

/* ---- DynQuantizedStorage (fuel-backend-contract/src/quantized.rs:29-103) ---- */
int frq_qstorage_dtype(const frq_qstorage *qs);
size_t frq_qstorage_block_size(const frq_qstorage *qs);
size_t frq_qstorage_size_in_bytes(const frq_qstorage *qs);
/* data(): host copy of the block bytes (synchronous). */
int frq_qstorage_data(const frq_qstorage *qs, void *host_dst, size_t nbytes);
/* device_ptr(): raw device address of the block bytes. */
int frq_qstorage_device_ptr(const frq_qstorage *qs, const void **out);
/* dequantize(elem_count) / dequantize_f16(elem_count) into a caller device
 * buffer of elem_count f32 / f16 values (to_float semantics). */
int frq_qstorage_dequantize(const frq_qstorage *qs, size_t elem_count, float *y_dev);
int frq_qstorage_dequantize_f16(const frq_qstorage *qs, size_t elem_count, uint16_t *y_dev);
/* quantize(src): from_float of elem_count f32 values on the device into this
 * storage (BlockQ4K::from_float k_quants.rs:1470-1528, BlockQ6K::from_float
 * :2005-2075, BlockQ8_0::from_float :629-658), bit-exact with the CPU
 * quantizer; elem_count must equal the storage's element count. */
int frq_qstorage_quantize(frq_qstorage *qs, const float *src_dev, size_t elem_count);
/* quantize_imatrix(src, imatrix_weights, n_per_row) and
 * quantize_imatrix_onto (fuel-backend-contract/src/quantized.rs:37-54;
 * CPU backend fuel-cpu-backend/src/quantized.rs:51-72): from_float_imatrix
 * of elem_count f32 values on the device (BlockQ4K k_quants.rs:1530-1593,
 * BlockQ6K :2077-2145), bit-exact with the CPU quantizer.  imatrix_host holds
 * n_per_row f32 importance weights (host memory, as the trait's slice); the
 * superblock with flat index s uses weights [(s % (n_per_row / 256)) * 256,
 * +256).  n_per_row must be a positive multiple of 256.  Q8_0 (and every
 * type without from_float_imatrix in the reference) gives FRQ_UNSUPPORTED. */
int frq_qstorage_quantize_imatrix(frq_qstorage *qs, const float *src_dev, size_t elem_count,
                                  const float *imatrix_host, size_t n_per_row);
/* fwd(self_shape = [n, k], input [m, k] contiguous f32) -> y [m, n] f32.
 * The trait method returns a fresh storage; here the caller passes the
 * output buffer (the host-side mirror allocates it). */
int frq_qstorage_fwd(const frq_qstorage *qs, size_t n, size_t k, const float *x_dev, size_t m,
                     float *y_dev);
/* fwd over an f16 input (DType::F16 branch of fwd, fuel-cpu-backend/src/
 * quantized.rs:127-137 -> matmul_t_f16 / matmul_f16, fuel-quantized/src/
 * k_quants.rs:2333-2374): x [m, k] f16 is widened exactly to f32, quantized
 * and dotted as in fwd; each output is rounded to f16 (f16::from_f32, round
 * to nearest even).  x 8-byte aligned, y 2-byte aligned. */
int frq_qstorage_fwd_f16(const frq_qstorage *qs, size_t n, size_t k, const uint16_t *x_dev, size_t m,
                         uint16_t *y_dev);

/* ---- KernelRef seam: (QMatMul, [F32, U32, F32]) ----
 * qmatmul_f32 wrapper semantics (fuel-dispatch/src/dispatch.rs:1638-1718 and
 * fuel-cpu-backend/src/byte_kernels.rs:4757-4830): act [batch, m, k] f32,
 * weight bytes = n * (k / block) blocks of `quant_type` (U32-typed storage,
 * 4-byte aligned), out [batch, m, n] f32 pre-allocated and fully overwritten.
 * Byte lengths are validated exactly as the CPU kernel does; a zero batch,
 * m or n is a no-op.  quant_type is the GgmlDType code (Q8_0 = 8,
 * Q4_K_M = Q4K = 12, Q6K = 14). */
int frq_qmatmul(frq_device *dev, int quant_type, size_t batch, size_t m, size_t n, size_t k,
                const float *act_dev, size_t act_bytes, const uint32_t *w_dev, size_t w_bytes,
                float *out_dev, size_t out_bytes);
/* frq_qmatmul without any device allocation.  No counterpart in the
 * reference: for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments
 * and checks as frq_qmatmul; the quantized activation rows and the split-K
 * partial sums live in a fixed 32 MiB device array per GPU instead of the
 * handle's growable workspace.  Results are bit-identical to frq_qmatmul's
 * when the plan's split-K partials fit beside the quantized rows; when they
 * do not, the K split is lowered until they fit (for 128 or more rows of
 * 16-byte aligned Q4_K blocks that can also select the wide-tile kernel), so
 * the f32 sums are added in another order and the results agree with
 * frq_qmatmul's within the path's tolerance (1e-3 of the output norm), not
 * in bits; frq_qmatmul_plan with noalloc = 1 reports the plan taken.  A call
 * whose quantized rows need more (about 1.14 * rows * k bytes for the
 * k-quants, 1.125 * rows * k for Q8_0) fails with status 4 (workspace).
 * Calls share that array: calls on one handle take turns (the handle's
 * lock), but calls that overlap on one GPU through two handles, or on two
 * streams, race. */
int frq_qmatmul_noalloc(frq_device *dev, int quant_type, size_t batch, size_t m, size_t n, size_t k,
                        const float *act_dev, size_t act_bytes, const uint32_t *w_dev, size_t w_bytes,
                        float *out_dev, size_t out_bytes);

/* ---- MoE mul_mat_id ----
 * Routing (LazyMoeRouter::route, fuel-core/src/lazy_nn/moe.rs:90-127;
 * MoeRouter::top_k_softmax and build_expert_batches, fuel-inference/src/
 * moe_routing.rs:252-275, 334-360): logits [t, e] f32 -> ids [t, topk] int32
 * (descending logit, ties to the lower expert id), w [t, topk] f32 softmax of
 * the picked logits, expert_offsets [e + 1], sorted_token_ids [t * topk]
 * (experts ascending, tokens ascending within an expert; the layout of the
 * CUDA routed-MMVQ FFI, fuel-cuda-backend/src/quantized.rs:138-144) and
 * sorted_slot [t * topk] (the flat entry token * topk + slot of each sorted
 * position; NULL to skip).  e <= 1024, 1 <= topk <= min(e, 64).  Device
 * pointers; asynchronous on the device stream. */
int frq_moe_route(frq_device *dev, const float *logits_dev, size_t t, size_t e, size_t topk,
                  int32_t *ids_dev, float *w_dev, int32_t *expert_offsets_dev,
                  int32_t *sorted_token_ids_dev, int32_t *sorted_slot_dev);
/* DynQuantizedStorage::indexed_moe_forward (fuel-backend-contract/src/
 * quantized.rs:82-95; the CUDA override was retired, fuel-cuda-backend/src/
 * quantized.rs:292-304): self = e experts of [n, k] blocks, expert-major;
 * x [t, x_slots, k] f32 with x_slots 1 (one row per token) or topk; ids
 * [t, topk] int32; y [t, topk, n] f32 with y[t][s] = W_{ids[t][s]} x[t][s or 0].
 * An id outside [0, e) gives a NaN row. */
int frq_indexed_moe_forward(const frq_qstorage *experts, size_t e, size_t n, size_t k,
                            const float *x_dev, size_t t, size_t x_slots, const int32_t *ids_dev,
                            size_t topk, float *y_dev);
/* The quantized expert layer (LazyMoeLayer::forward, lazy_nn/moe.rs:296-348):
 * route logits [t, e] as frq_moe_route, then for every expert
 * y_e = down(silu(gate(x_sel)) * up(x_sel)) over its routed rows and
 * out[t] = sum of w_{t,e} * y_e[t] in ascending expert order.  w_gate and
 * w_up hold e experts of [ffn, d] blocks, w_down e experts of [d, ffn] blocks
 * (ggml_dtype, expert-major); x [t, d] f32, out [t, d] f32. */
int frq_moe_ffn(frq_device *dev, int ggml_dtype, size_t t, size_t d, size_t ffn, size_t e, size_t topk,
                const float *x_dev, const float *logits_dev, const void *w_gate_dev, const void *w_up_dev,
                const void *w_down_dev, float *out_dev);

/* ---- decode-step fusions around the QMatMul ----
 * The QMatMul (k_quants.rs:2284-2331) with its neighbours in fuel's LLaMA
 * layer (fuel-core/src/lazy.rs:7363-7440) fused into one mat-vec launch:
 *   a = x                                   (plain), or
 *   a = (x * rsqrt(mean(x^2) + eps)) * gain (rms_norm_last_dim_f32 and
 *       apply_affine_rms_norm, byte_kernels.rs:2339-2368, lazy.rs:10330-10346;
 *       rms_gain_dev != NULL), or
 *   a = silu(x) * x2 = x / (1 + exp(-x)) * x2 (the SwiGLU input,
 *       lazy.rs:7433-7434; x2_dev != NULL),
 *   y[r, :] = W a(x[r, :])  or, with accumulate, y[r, :] += W a(x[r, :])
 *       (the residual adds, lazy.rs:7426, 7439).
 * Rows r < m of x (and x2) are ldx floats apart, of y ldy apart.  x, x2 and
 * gain must be 16-byte aligned with ldx % 4 == 0.  Asynchronous.  With one
 * row (the decode step) it is one mat-vec launch that allocates nothing, so
 * it may be captured into a HIP graph; with m >= 2 rows of Q4K / Q6K
 * weights the rows a(x) are formed and quantized once into the device
 * workspace (grown on demand, as frq_qmatmul's) and the batched int8-MFMA
 * kernels read every weight block once, the residual added in their
 * epilogue (the batched prompt pass). */
int frq_qmatmul_fused(frq_device *dev, int ggml_dtype, size_t m, size_t n, size_t k, const void *w_dev,
                      const float *x_dev, size_t ldx, const float *x2_dev, const float *rms_gain_dev,
                      float rms_eps, int accumulate, float *y_dev, size_t ldy);
/* Two QMatMuls of the same activation rows in one launch (the [q|k] and v
 * projections of a layer, lazy.rs:7384-7386): y1[r, :] = W1 a(x[r, :]) and
 * y2[r, :] = W2 a(x[r, :]) with a() the plain or RMS-normalized activation of
 * frq_qmatmul_fused; W1 / W2 are Q4K or Q6K (k % 256 == 0, k <= 16384); y1 /
 * y2 rows are n1 / n2 floats.  Asynchronous; with one row capturable (no
 * allocation), with m >= 2 the rows are normalized and quantized once into
 * the device workspace for both batched matmuls. */
int frq_qmatmul_fused_pair(frq_device *dev, size_t m, size_t k, const float *x_dev, size_t ldx,
                           const float *rms_gain_dev, float rms_eps, int dtype1, size_t n1, const void *w1_dev,
                           float *y1_dev, int dtype2, size_t n2, const void *w2_dev, float *y2_dev);
/* The gated FFN input of LlamaModel::apply_layer (lazy.rs:7436-7442:
 * gate = a.qmatmul(W_gate), up = a.qmatmul(W_up), silu(gate) * up with
 * silu(g) = g / (1 + exp(-g)), byte_kernels.rs silu):
 * y[m][n] = silu(W_gate . a_m) * (W_up . a_m), a_m = rms_norm(x_m) * rms_gain
 * (or x_m when rms_gain_dev is NULL), both matrices [n, k] blocks of dtype.
 * One launch; each output's gate and up rows are reduced by the same
 * wavefront, so the product is formed where both sums are and only n
 * values are written.  Bit-identical to the two outputs of
 * frq_qmatmul_fused (or the pair form) followed by the SwiGLU input stage
 * of frq_qmatmul_fused (x2). */
int frq_qmatmul_fused_glu(frq_device *dev, int dtype, size_t m, size_t n, size_t k, const void *w_gate_dev,
                          const void *w_up_dev, const float *x_dev, size_t ldx, const float *rms_gain_dev,
                          float rms_eps, float *y_dev, size_t ldy);
/* Decode attention of one token (lazy.rs:7391-7423 at seq = 1 with a KV
 * cache): q and k of qk_dev = [q | k] (n_heads * head_dim each) are rotated
 * (rope_f32 rotate-half, byte_kernels.rs:1885-1964, with the rows `pos` of
 * the [max_ctx, head_dim] tables of build_rope_tables, fuel-graph/src/
 * lib.rs:10808-10868), k and v are rounded to f16 and written at row `pos` of
 * the caches [n_heads, max_ctx, head_dim], then per head
 * out = softmax((q . k_j) * scale over j <= pos) . v_j.  pos is read from
 * device memory (*pos_dev) so that a captured call serves every position.
 * n_kv_heads = n_heads; head_dim = 128.  work_dev: at least
 * frq_attention_decode_workspace() bytes of scratch for the per-split
 * partials (no initialization needed).  A pos outside [0, max_ctx) gives NaN
 * outputs and writes no cache row. */
size_t frq_attention_decode_workspace(size_t n_heads, size_t max_ctx);
int frq_attention_decode(frq_device *dev, size_t n_heads, size_t head_dim, size_t max_ctx, const float *qk_dev,
                         const float *v_dev, const float *rope_cos_dev, const float *rope_sin_dev,
                         uint16_t *k_cache_dev, uint16_t *v_cache_dev, const int32_t *pos_dev, float scale,
                         void *work_dev, size_t work_bytes, float *out_dev);
/* frq_attention_decode followed by the attention output projection with the
 * residual add, y_dev[n_out] += W_o . attn (lazy.rs:7427-7434: o_proj then
 * the residual).  When the context needs at most 8 splits (the split count
 * is max(ceil(256 / n_heads), ceil(max_ctx / 128)): 32 heads up to
 * max_ctx 1024) this is two launches instead of three: the per-split
 * partials are merged inside the o-projection mat-vec (each workgroup merges
 * its activation row while its first weight rows load) instead of by a
 * separate kernel; otherwise the merge kernel writes into the workspace's
 * tail first.  w_o_dev: [n_out, n_heads * head_dim] blocks of o_dtype (Q8_0, Q4_K,
 * Q6_K); n_heads * head_dim must be a multiple of 256.  Same caches, appends
 * and workspace as frq_attention_decode (work_dev 16-byte aligned here); the
 * result is bit-identical to frq_attention_decode then frq_qmatmul_fused with
 * accumulate = 1.  A pos outside [0, max_ctx) makes the attention NaN, as
 * there. */
int frq_attention_decode_oproj(frq_device *dev, size_t n_heads, size_t head_dim, size_t max_ctx,
                               const float *qk_dev, const float *v_dev, const float *rope_cos_dev,
                               const float *rope_sin_dev, uint16_t *k_cache_dev, uint16_t *v_cache_dev,
                               const int32_t *pos_dev, float scale, void *work_dev, size_t work_bytes, int o_dtype,
                               const void *w_o_dev, size_t n_out, float *y_dev);
/* ---- prefill: row kernels of a batched prompt pass ----
 * LlamaModel::apply_layer (lazy.rs:7363-7446) at seq = m: the projections
 * are frq_qmatmul calls (int8 MFMA for m >= 16) and these kernels run
 * between them.  Row-major buffers with leading dimensions in elements. */
/* y[r] = (x[r] * (1 / sqrt(sum(x[r]^2) / k + eps))) * gain, per row
 * (rms_norm_last_dim_f32, byte_kernels.rs:2339-2368, and the affine gain,
 * lazy.rs:10330-10346; the sum of squares is a tree, sequential there). */
int frq_rms_norm_rows(frq_device *dev, size_t m, size_t k, const float *x_dev, size_t ldx, const float *gain_dev,
                      float eps, float *y_dev, size_t ldy);
/* Row r of qk_dev = [q | k] (n_heads * head_dim each) and of v_dev, at
 * position pos0 + r: q and k rotated (rope_f32 rotate-half,
 * byte_kernels.rs:1885-1964, with rows of the [max_ctx, head_dim] tables), q
 * written back in place, k and v rounded to f16 into cache row pos0 + r of
 * every head ([n_heads, max_ctx, head_dim] caches, as frq_attention_decode
 * appends).  head_dim = 128. */
int frq_rope_append_rows(frq_device *dev, size_t m, size_t n_heads, size_t head_dim, size_t max_ctx, float *qk_dev,
                         size_t ldqk, const float *v_dev, size_t ldv, const float *rope_cos_dev,
                         const float *rope_sin_dev, size_t pos0, uint16_t *k_cache_dev, uint16_t *v_cache_dev);
/* Causal attention of m query rows (rotated q, [m, n_heads * head_dim]) at
 * positions pos0 .. pos0 + m - 1 over the f16 cache rows 0 .. each row's
 * position (lazy.rs:7415-7425: scores * scale plus the strict-causal mask,
 * softmax_last_dim, times V), one pass with a running maximum.  The rows
 * pos0 .. pos0 + m - 1 must already be in the caches (frq_rope_append_rows). */
int frq_attention_prefill(frq_device *dev, size_t m, size_t n_heads, size_t head_dim, size_t max_ctx,
                          const float *q_dev, size_t ldq, const uint16_t *k_cache_dev, const uint16_t *v_cache_dev,
                          size_t pos0, float scale, float *out_dev, size_t ldo);
/* h[r][i] = silu(gu[r][i]) * gu[r][f + i], silu(g) = g / (1 + exp(-g))
 * (lazy.rs:7442 on the [gate | up] output of one stacked projection). */
int frq_swiglu_rows(frq_device *dev, size_t m, size_t f, const float *gu_dev, size_t ldgu, float *h_dev, size_t ldh);
/* y[i] += x[i] for i < n (the residual adds, lazy.rs:7434, 7446). */
int frq_add(frq_device *dev, size_t n, const float *x_dev, float *y_dev);
/* out[r] = table[ids[r]] (rows of dim floats; an id outside [0, rows) reads
 * row 0): the prompt's embedding rows. */
int frq_gather_rows(frq_device *dev, const float *table_dev, size_t rows, size_t dim, const int32_t *ids_dev,
                    size_t m, float *out_dev);
/* Greedy next token and its embedding: next = tokens[pos + 1] while
 * pos + 1 < *prompt_len_dev, else the first-index argmax of logits [vocab]
 * (argmax_dim_f32, byte_kernels.rs:8246-8261), stored at tokens[pos + 1]
 * (when pos + 1 < tokens_cap); x = table[next] ([vocab, dim] f32, dim % 4 == 0);
 * *pos_dev += 1.  The prompt length is read on the device, like the position,
 * so one captured step serves every prompt.  Asynchronous, capturable. */
int frq_argmax_embed(frq_device *dev, const float *logits_dev, size_t vocab, const float *table_dev, size_t dim,
                     int32_t *tokens_dev, size_t tokens_cap, const int32_t *prompt_len_dev, int32_t *pos_dev,
                     float *x_dev);

/* ---- integer taps (build-internal parity probes; no reference counterpart) ----
 * Quantize rows of f32 activations into fuel's activation blocks
 * (BlockQ8K::from_float k_quants.rs:2230-2267, BlockQ8_0::from_float
 * :629-658), written in the reference byte layout [rows, k/blk] blocks. */
int frq_quantize_q8k(frq_device *dev, const float *x_dev, size_t rows, size_t k, void *blocks_dev);
int frq_quantize_q8_0(frq_device *dev, const float *x_dev, size_t rows, size_t k, void *blocks_dev);
/* The kernels frq_qmatmul (noalloc = 0) or frq_qmatmul_noalloc (noalloc = 1)
 * runs for `rows` activation rows of an [n, k] weight of quant_type whose
 * blocks start at w_dev (only its 16-byte alignment matters): *path is 0
 * (the fused quantize + mat-vec, one row), 1 (the mat-vec over 2-4 rows
 * quantized in LDS), 2 (the few-row int8-MFMA kernel) or 3 (the tiled
 * int8-MFMA GEMM); for path 3 *kind is the tile kernel and *ksplit the number
 * of K splits summed in split order, else -1 and 1.  Build-internal tap with
 * no counterpart in the reference: the plan (and so the f32 summation order)
 * is a function of these arguments and the device's CU count alone, which
 * the reference's bit_stable_on_same_hardware (fuel-dispatch/src/fused.rs:
 * 1319-1330) requires. */
int frq_qmatmul_plan(frq_device *dev, int quant_type, size_t rows, size_t n, size_t k, const void *w_dev,
                     int noalloc, int *path, int *kind, int *ksplit);
/* Per-(row m, weight row n, block b) integer sums of the block dot product
 * (vec_dot_unopt's integer stage): isum/msum [m, n, k/blk] int32.  The
 * activations are quantized on the device from x_dev first. */
int frq_block_isums(frq_device *dev, int ggml_dtype, size_t m, size_t n, size_t k,
                    const void *w_dev, const float *x_dev, int32_t *isum_dev, int32_t *msum_dev);

/* ---- synthetic inputs (no reference counterpart: seeded test/bench data) ----
 * Philox-4x32-10 words in fuel's RandomBits layout (fuel-cpu-kernels/src/
 * philox.rs:91-133): element i = lane i%4 of the block at counter
 * [(start+i)/4 lo, hi, base, stream], key = seed. */
int frq_fill_random_bits(frq_device *dev, uint32_t *y_dev, size_t n, uint64_t start, uint64_t seed,
                         uint32_t base, uint32_t stream);
/* N(mean, std) by Box-Muller over the same words (counter base 0). */
int frq_fill_normal(frq_device *dev, float *y_dev, size_t n, uint64_t seed, uint32_t stream, float mean,
                    float std);

/* ---- measurement helper (no reference counterpart) ----
 * A read-only streaming kernel over `bytes` of device memory (16-byte aligned,
 * a multiple of 16): wg_per_cu * CUs workgroups of 256 threads, `unroll`
 * (1, 2, 4 or 8) 16-byte loads per thread in flight (non-temporal loads when
 * `nontemporal` is nonzero), nothing written but sink[0] in the rare case the
 * loaded words XOR to a fixed constant.  Times the HBM read ceiling of one
 * launch of that size, the bound the mat-vec's roofline fraction is read
 * against. */
int frq_probe_read(frq_device *dev, const void *src_dev, size_t bytes, int wg_per_cu, int unroll, int nontemporal,
                   uint32_t *sink_dev);

/* ---- GGUF files (host-side reader + upload) ----
 * frq_gguf_open maps the file read-only and parses its header exactly as
 * fuel_formats::gguf::Content::read (fuel-formats/src/gguf.rs:378-461) over
 * fuel-core's mmap (fuel-core/src/quantized/gguf_mmap.rs:44-79): magic
 * "GGUF" (either byte order), versions 1-3 (u32 counts and lengths in v1, u64
 * after), metadata values of types 0-12 (nested arrays included; strings lose
 * trailing NULs and invalid UTF-8 becomes U+FFFD), tensor infos with their
 * dims reversed (outermost first, as fuel's Shape), GgmlDType codes of
 * GgmlDType::from_u32, and tensor_data_offset = position rounded up to
 * general.alignment (u8/u16/u32 or non-negative i8/i16/i32; else 32).  A
 * repeated metadata key or tensor name keeps its first position and the last
 * value.  Errors (FRQ_INVALID) carry the reference's messages ("unknown magic
 * ...", "unrecognized value-type ...", "unexpected bool value ...", "unknown
 * dtype for tensor ...").  The handle owns the mapping until frq_gguf_close. */
typedef struct frq_gguf frq_gguf;
typedef struct frq_gguf_value frq_gguf_value;
int frq_gguf_open(const char *path, frq_gguf **out);
int frq_gguf_close(frq_gguf *g);
int frq_gguf_version(const frq_gguf *g);
uint64_t frq_gguf_tensor_data_offset(const frq_gguf *g);
size_t frq_gguf_tensor_count(const frq_gguf *g);
/* Tensor `index` (file order): name, GgmlDType code, dims (outermost first,
 * at most dims_cap written), offset relative to tensor_data_offset, and its
 * byte length elem_count / block_size * type_size (the slice the lazy loaders
 * take, fuel-core/src/lazy_quantized_llama.rs:251-260). */
int frq_gguf_tensor_info(const frq_gguf *g, size_t index, const char **name, int *ggml_dtype, size_t *n_dims,
                         uint64_t *dims, size_t dims_cap, uint64_t *offset, uint64_t *nbytes);
int frq_gguf_find_tensor(const frq_gguf *g, const char *name, size_t *index);
/* Host view of a tensor's bytes inside the mapping (bounds-checked). */
int frq_gguf_tensor_data(const frq_gguf *g, size_t index, const void **host, uint64_t *nbytes);
/* QuantizedDeviceKernels::load_quantized(dtype, bytes) of one tensor: its
 * blocks uploaded verbatim ([out, in] block order) into a new storage
 * (Q8_0 / Q4_K / Q6_K / Q8_K tensors). */
int frq_gguf_load_quantized(frq_device *dev, const frq_gguf *g, size_t index, frq_qstorage **out);
/* Metadata in file order and by key; values are read through the accessors
 * below (the Value enum, gguf.rs:164-375): value_type is the format's code,
 * value_scalar yields the raw payload of a scalar (unsigned types and bool in
 * u, signed in i, f32/f64 in f), value_u64 follows Value::to_u64 (u64, or u8 /
 * u16 / u32 / bool upcast), arrays are walked with value_array /
 * value_array_at. */
size_t frq_gguf_meta_count(const frq_gguf *g);
int frq_gguf_meta_at(const frq_gguf *g, size_t index, const char **key, const frq_gguf_value **value);
int frq_gguf_meta_find(const frq_gguf *g, const char *key, const frq_gguf_value **value);
int frq_gguf_value_type(const frq_gguf_value *v);
int frq_gguf_value_scalar(const frq_gguf_value *v, uint64_t *u, int64_t *i, double *f);
int frq_gguf_value_u64(const frq_gguf_value *v, uint64_t *out);
int frq_gguf_value_string(const frq_gguf_value *v, const char **s, size_t *len);
int frq_gguf_value_array(const frq_gguf_value *v, size_t *len);
int frq_gguf_value_array_at(const frq_gguf_value *v, size_t j, const frq_gguf_value **elem);

#ifdef __cplusplus
}
#endif
#endif
