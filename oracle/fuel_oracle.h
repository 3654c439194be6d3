/*
 * fuel_oracle.h -- CPU restatement of fuel's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (fuel_amd/, include/)
 * includes, links or calls this code.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg use it, as the checker / CPU baseline.
 *
 * Every function restates the named reference function in
 * /root/reference/fuel-quantized/src (k_quants.rs, avx.rs, utils.rs),
 * fuel-cpu-kernels/src/philox.rs and fuel-inference/src/moe_routing.rs.
 * The reference is Rust and cannot be compiled in this image (no cargo or
 * rustc), so there is no oracle/_ref build; the restatement is pinned by the
 * checks listed in tests/test_oracle_*.py.
 */
#ifndef FUEL_ORACLE_H
#define FUEL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FO_QK_K 256
#define FO_QK8_0 32

/* Block layouts: byte-exact with k_quants.rs:92-98 (BlockQ8_0),
 * :129-138 (BlockQ4K), :152-160 (BlockQ6K), :162-169 (BlockQ8K).
 * f16 fields are kept as raw IEEE binary16 bit patterns. */
typedef struct {
    uint16_t d;
    int8_t qs[32];
} fo_block_q8_0;

typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[128];
} fo_block_q4k;

typedef struct {
    uint8_t ql[128];
    uint8_t qh[64];
    int8_t scales[16];
    uint16_t d;
} fo_block_q6k;

typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} fo_block_q8k;

/* GgmlDType codes (fuel-ir/src/quantized.rs:36-76). */
enum { FO_Q8_0 = 8, FO_Q4K = 12, FO_Q6K = 14, FO_Q8K = 15 };

size_t fo_type_size(int ggml_dtype);
size_t fo_block_size(int ggml_dtype);

/* ---- f16 <-> f32 (the `half` crate's to_f32 / from_f32, RNE) ---- */
float fo_f16_to_f32(uint16_t h);
uint16_t fo_f32_to_f16(float f);

/* ---- Philox-4x32-10 and seeded synthetic inputs (philox.rs:47-135) ---- */
void fo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
void fo_random_bits_fill(uint32_t *dst, size_t n, uint64_t start_index, uint64_t seed,
                         uint32_t base, uint32_t stream);
/* N(mean, std) via Box-Muller over Philox words; element i uses Philox block
 * i/4 (words 2p, 2p+1 with p = (i%4)/2) and takes cos for even i, sin for odd. */
void fo_normal_fill(float *dst, size_t n, uint64_t seed, uint32_t stream, float mean, float std);
/* Uniform integers in [0, bound): (word * bound) >> 32 over random_bits. */
void fo_uniform_u32_fill(uint32_t *dst, size_t n, uint64_t seed, uint32_t stream, uint32_t bound);

/* ---- activation quantizers (from_float) ---- */
void fo_quantize_q8k(const float *x, size_t k, fo_block_q8k *y);   /* k_quants.rs:2230-2267 */
void fo_quantize_q8_0(const float *x, size_t k, fo_block_q8_0 *y); /* k_quants.rs:629-658 */

/* ---- weight quantizers (from_float) ---- */
void fo_quantize_q4k(const float *x, size_t k, fo_block_q4k *y);   /* k_quants.rs:1470-1528 */
void fo_quantize_q6k(const float *x, size_t k, fo_block_q6k *y);   /* k_quants.rs:2005-2075 */
/* from_float_imatrix (k_quants.rs:1530-1593 Q4_K, 2077-2145 Q6_K): importance
 * weights imatrix[n_per_row], the flat superblock s using column block
 * s % (n_per_row / 256).  Returns -1 for other types or a bad n_per_row. */
int fo_quantize_imatrix(int ggml_dtype, const float *x, size_t k, const float *imatrix, size_t n_per_row, void *y);
/* Row-parallel (OpenMP) wrappers over the per-row quantizers above;
 * rows are independent so the bytes are identical to the serial call. */
void fo_quantize_rows(int ggml_dtype, const float *x, size_t rows, size_t k, void *y);

/* ---- dequantizers (to_float) ---- */
void fo_dequantize(int ggml_dtype, const void *blocks, size_t k, float *y);

/* ---- block dot products ---- */
/* Scalar vec_dot_unopt restatements (exact f32 operation order). */
float fo_vec_dot_q4k_unopt(size_t k, const fo_block_q4k *w, const fo_block_q8k *a);
float fo_vec_dot_q6k_unopt(size_t k, const fo_block_q6k *w, const fo_block_q8k *a);
float fo_vec_dot_q8_0_unopt(size_t k, const fo_block_q8_0 *w, const fo_block_q8_0 *a);
/* AVX2 vec_dot restatements (avx.rs), identical lane partition and f32
 * order; return NaN when the host lacks AVX2+FMA. */
float fo_vec_dot_q4k_avx2(size_t k, const fo_block_q4k *w, const fo_block_q8k *a);
float fo_vec_dot_q6k_avx2(size_t k, const fo_block_q6k *w, const fo_block_q8k *a);
float fo_vec_dot_q8_0_avx2(size_t k, const fo_block_q8_0 *w, const fo_block_q8_0 *a);
int fo_have_avx2(void);

/* Per-superblock integer sums (the bit-exact stage of a8-a10):
 * isum[b] = sum_j sc_j * sum_l q*q8, msum[b] = sum_g bsums_g * m_{g/2}
 * (Q4K only; zero for the others). */
void fo_block_isums(int ggml_dtype, size_t k, const void *w_row, const void *a_row,
                    int32_t *isum, int32_t *msum);

/* ---- matmul<T> (k_quants.rs:2284-2331) ----
 * x [m,k] f32, w [n, k/blk] blocks, y [m,n] f32.  `use_avx2` selects the
 * AVX2 vec_dot (what target-cpu=native selects) or vec_dot_unopt.
 * `threads` <= 0 means OpenMP default.  Returns 0 or a status code. */
int fo_matmul(int ggml_dtype, size_t m, size_t k, size_t n, const float *x, const void *w,
              float *y, int use_avx2, int threads);

/* qmatmul_generic_f32 (fuel-cpu-backend/src/byte_kernels.rs:4757-4830):
 * byte-length validation then batched matmul.  Returns 0 ok, 2 invalid. */
int fo_qmatmul_bytes(int ggml_dtype, size_t batch, size_t m, size_t n, size_t k,
                     const float *act, size_t act_bytes, const void *w, size_t w_bytes,
                     float *out, size_t out_bytes, int use_avx2, int threads);

/* ---- MoE routing (moe_routing.rs:252-275, 334-360; lazy_nn/moe.rs:90-127) ----
 * logits [t, e]; ids [t, topk] (descending logit, ties -> lower expert id);
 * w [t, topk] softmax over the picked logits; expert_offsets [e+1];
 * sorted_token_ids [t*topk] (token ids ascending within each expert);
 * sorted_slot [t*topk] = the (token, slot) flat index each entry came from. */
void fo_moe_route(const float *logits, size_t t, size_t e, size_t topk, int32_t *ids, float *w,
                  int32_t *expert_offsets, int32_t *sorted_token_ids, int32_t *sorted_slot);

/* Expert FFN over the routed rows (lazy_nn/moe.rs:204-235, 296-348):
 * out[t] = sum over the token's experts, in ascending expert order, of
 * w_{t,e} * down_e(silu(gate_e(x_t)) * up_e(x_t)).  Weights are Q4K (or
 * any supported dtype) with gate/up [ffn, d] and down [d, ffn] per expert,
 * concatenated expert-major. */
int fo_moe_ffn(int ggml_dtype, size_t t, size_t d, size_t ffn, size_t e, size_t topk,
               const float *x, const int32_t *ids, const float *w, const void *w_gate,
               const void *w_up, const void *w_down, float *out, int use_avx2, int threads);

/* ---- LLaMA decoder pieces (fuel-core/src/lazy.rs:7363-7440) ----
 * rms_norm_last_dim_f32 (fuel-cpu-backend/src/byte_kernels.rs:2339-2368)
 * followed by the affine gain (apply_affine_rms_norm, lazy.rs:10330-10346):
 * y = (x * (1 / sqrt(sum(x^2) * (1/dim) + eps))) * gain, per row. */
void fo_rms_norm(const float *x, const float *gain, size_t rows, size_t dim, float eps, float *y);
/* build_rope_tables (fuel-graph/src/lib.rs:10808-10868): cos/sin
 * [seq, head_dim] for positions start_pos.., computed in f64. */
void fo_rope_tables(double base, size_t start_pos, size_t seq, size_t head_dim, float *cos_t, float *sin_t);
/* rope_f32 rotate-half (byte_kernels.rs:1885-1964): x [outer, seq, head_dim],
 * tables [seq, head_dim]. */
void fo_rope(const float *x, const float *cos_t, const float *sin_t, size_t outer, size_t seq, size_t head_dim,
             float *y);
/* One query per head against cached keys / values [heads, stride, head_dim]
 * (first n_ctx rows): scores = (q . k_j) * scale (lazy.rs:7416-7420),
 * softmax_last_dim_f32 (byte_kernels.rs:2259-2305), out = sum_j p_j v_j
 * (lazy.rs:7422). q / out: [heads, head_dim]. */
void fo_attention_decode(const float *q, const float *k, const float *v, size_t heads, size_t n_ctx, size_t stride,
                         size_t head_dim, float scale, float *out);
/* argmax_dim_f32 over one row (byte_kernels.rs:8178-8261): first element
 * taken, then strictly greater values. */
size_t fo_argmax(const float *x, size_t n);

#ifdef __cplusplus
}
#endif
#endif
