// Host-side launchers of the device kernels (one translation unit each).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace frq {

// quantize.hip
hipError_t launch_quantize_q8k(const float* x, int rows, int K, ActView act, uint8_t* aos,
                               hipStream_t s);
// Q8K rows of silu(g) * u with g = x[m][0, K) and u = x[m][K, 2K) (row stride ldx).
hipError_t launch_quantize_q8k_swiglu(const float* x, int ldx, int rows, int K, ActView act, hipStream_t s);
// The activation rows of a fused QMatMul, formed before the Q8K quantize: x
// (row stride ldx); with x2, silu(x) * x2 (x2 rows of the same stride); with
// gain, rms_norm(x) * gain (eps inside the root; the fused mat-vec prologue's
// arithmetic).  x2 and gain are exclusive; gain needs K <= 32768.
struct ActSrc {
    const float* x;
    int ldx;
    const float* x2;
    const float* gain;
    float eps;
};
bool quantize_src_supported(const ActSrc& src, int K);
hipError_t launch_quantize_q8k_src(const ActSrc& src, int rows, int K, ActView act, hipStream_t s);
hipError_t launch_quantize_q8_0(const float* x, int rows, int K, ActView act, uint8_t* aos,
                                hipStream_t s);
// Q8K rows of f16 activations (widened exactly to f32 first).
hipError_t launch_quantize_q8k_h(const uint16_t* x, int rows, int K, ActView act, hipStream_t s);
hipError_t launch_quantize_q8_0_h(const uint16_t* x, int rows, int K, ActView act, hipStream_t s);

// mmvq.hip: y[m, n] = sum_b blockdot(W[n, b], quantize(x[m])_b) for rows m < M,
// activation quantization fused into the kernel.
hipError_t launch_qmv(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K,
                      int ldy, hipStream_t s, int num_cus);
// The same over f16 activations and f16 outputs (matmul_f16).
hipError_t launch_qmv_half(int dtype, const uint8_t* w, const uint16_t* x, uint16_t* y, int M, int N, int K, int ldy,
                           hipStream_t s, int num_cus);

// Options of the generalized mat-vec.
// Indexed (MoE mul_mat_id): launch row m reads activation row x_row[m] (or
// m / x_div when x_row is null; stride ldx floats) and the weights of expert
// w_sel[m] (expert_bytes apart; an id outside [0, n_experts) yields a NaN
// output row and reads no weights).  Output rows n >= n_split come from W2
// instead of W (gate|up in one launch).
// Both modes: with x2 set the activation is silu(x) * x2, the SwiGLU input of
// the down projection (x2 indexed like x).
// Fused (decode step): activation row m at x + m * ldx; with rms_gain set it
// is first RMS-normalized with the affine gain, (x * rsqrt(mean(x^2) + eps)) *
// gain; with accumulate set the output is added to y (residual stream).
struct QmvOpts {
    const int* x_row;
    int x_div;
    int ldx;
    const int* w_sel;
    int n_experts;
    size_t expert_bytes;
    const uint8_t* w2;
    int n_split;
    const float* x2;
    const float* rms_gain;
    float rms_eps;
    int accumulate;
    // attention-merging mode (launch_qmv_attn): x holds the decode-attention
    // split partials, M = 1
    int attn_nsplit;
    int attn_max_ctx;
    const int* attn_pos;
    // routing mode (launch_qmv_indexed_route): launch row m is slot m % x_div
    // of token m / x_div, whose expert the workgroup picks itself from the
    // token's router logits (n_experts <= 128 of them, x_div = topk); the
    // workgroups with blockIdx.x = 0 store the picks and their weights
    const float* route_logits;
    int* route_ids;
    float* route_w;
    // several activation rows per workgroup (plain mode): the rows in all
    int rows;
};
hipError_t launch_qmv_indexed(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                              const QmvOpts& ix, hipStream_t s, int num_cus);
// The plain mat-vec for a few rows of the k-quants: every workgroup quantizes
// MR (2 or 4) rows into LDS and reduces each weight row against all of them
// while it is in registers (one weight pass per MR rows, no quantize launch).
constexpr int QMV_MULTI_MAX_ROWS = 4;
bool qmv_multi_supported(int dtype, int M, int N, int K);
hipError_t launch_qmv_multi(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                            hipStream_t s, int num_cus);
hipError_t launch_qmv_indexed_route(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K,
                                    int ldy, const QmvOpts& ix, hipStream_t s, int num_cus);
constexpr int QMV_ROUTE_MAX_EXPERTS = 128;
hipError_t launch_qmv_fused(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                            const QmvOpts& o, hipStream_t s, int num_cus);
// y [M, N] = silu(Wg a(x)) * (Wu a(x)), a(x) as launch_qmv_fused (RMS norm
// from o; no x2, no accumulate).
hipError_t launch_qmv_glu(int dtype, const uint8_t* w_gate, const uint8_t* w_up, const float* x, float* y, int M, int N,
                          int K, int ldy, const QmvOpts& o, hipStream_t s, int num_cus);
// y [N] (+)= W a where a [K = heads * ATTN_HEAD_DIM] is the merge of the
// decode-attention partials in `part` (attn_decode_work layout, o.attn_*
// set): the merge runs in each workgroup's activation stage.
hipError_t launch_qmv_attn(int dtype, const uint8_t* w, const float* part, float* y, int N, int K, const QmvOpts& o,
                           hipStream_t s, int num_cus);
// Two fused mat-vecs of the same activation rows (ldx apart, optional RMS
// norm from `o`) in one launch: y1 [M, n1] = W1 a(x), y2 [M, n2] = W2 a(x);
// Q4K / Q6K weights, K <= 16384.
bool qmv_pair_supported(int dt1, int dt2, int K);
hipError_t launch_qmv_pair(int dt1, const uint8_t* w1, float* y1, int n1, int dt2, const uint8_t* w2, float* y2,
                           int n2, const float* x, int M, int K, const QmvOpts& o, hipStream_t s, int num_cus);

// moe.hip: top-k softmax routing of logits [T, E] (ids/w [T, topk]), the
// expert batches of the routed entries (counting sort: expert_offsets [E+1],
// per sorted position the token, the flat (token, slot) entry and the expert,
// per entry its sorted position), and the combine of the per-position expert
// outputs yd [P, d] back onto the tokens in ascending expert order.
constexpr int MOE_MAX_EXPERTS = 1024;
constexpr int MOE_MAX_TOPK = 64;
hipError_t launch_moe_route(const float* logits, int T, int E, int topk, int* ids, float* w, hipStream_t s);
// With tile_bm > 0 the batches kernel also writes the tile table of a grouped
// matmul: tiles of tile_bm sorted rows, expert by expert (tile_expert,
// tile_row0, ntiles[0] = count; at most P / tile_bm + E tiles).
struct MoeTiles {
    int bm;
    int* tile_expert;
    int* tile_row0;
    int* ntiles;
};
hipError_t launch_moe_batches(const int* ids, int P, int E, int topk, int* offsets, int* sorted_token,
                              int* sorted_slot, int* entry_expert, int* entry_pos, const MoeTiles& tiles,
                              hipStream_t s);
hipError_t launch_moe_combine(const float* yd, const int* ids, const float* w, const int* entry_pos, int T, int topk,
                              int d, float* out, hipStream_t s);
// The down projection and the combine in one launch for the mat-vec path:
// out [T, d] from gu [T * topk, 2 ffn] (gate | up per routed entry, routing
// order), ids / w [T, topk] and the experts' down matrices [d, ffn]
// (expert_bytes apart).  Supported for Q4_K / Q6_K / Q8_0 when an entry's
// blocks fit 32 lanes and topk and the activation rows fit its instantiations.
bool moe_down_combine_supported(int dtype, int topk, int ffn);
hipError_t launch_moe_down_combine(int dtype, const uint8_t* w, size_t expert_bytes, int E, const float* gu,
                                   const int* ids, const float* wts, int T, int topk, int ffn, int d, float* out,
                                   hipStream_t s, int num_cus);
// mmq_skinny.hip: int8-MFMA matmul for a few rows (activations already
// quantized into the workspace, Q8K for the k-quants, Q8_0 for Q8_0), each
// weight block read once for every row group of up to 32 rows; y [M, N] with
// row stride ldy.  K must be a multiple of 256.
bool mmq_skinny_supported(int dtype, int K);
hipError_t launch_mmq_skinny(int dtype, const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy,
                             int num_cus, hipStream_t s, int out_mode = 0);
// mmq.hip: int8-MFMA matmul for M >= 16 over activations already quantized
// into the workspace (quantize_q8k), y [M, N] with row stride ldy.
// mmq_plan picks the kernel (tile shape; the LDS-DMA staging only for 16-byte
// aligned Q4_K blocks) and the K split on the host; part_elems is the number
// of f32 split-K partial sums launch_mmq needs in `part` (0 without a split).
// out_mode (common.hpp): OUT_F16 stores f16 outputs (round to nearest even
// of the f32 sums), OUT_ACC adds the sums to the f32 values already in y.
bool mmq_supported(int dtype);
struct MmqPlan {
    int kind;           // kernel instantiation
    int ks;             // K splits (1: none)
    size_t part_elems;  // split partial sums: ks * M * N, or 0
};
// max_part_elems caps the partials: the K split is lowered until they fit.
MmqPlan mmq_plan(int dtype, const void* w, int M, int N, int K, int num_cus, size_t max_part_elems = ~(size_t)0);
hipError_t launch_mmq(const MmqPlan& plan, int dtype, const uint8_t* w, ActView act, float* y, float* part, int M,
                      int N, int K, int ldy, hipStream_t s, int out_mode = 0);

// Grouped (MoE) int8-MFMA matmul: workgroup x takes tile x of the tile table
// (rows [tile_row0, expert end) of one expert, up to bm of them); its weights
// are expert e's (expert_bytes apart), columns n >= n_split read w2 instead
// (gate|up in one launch), activation row m is x_row[m] (null: m).
struct MmqGroup {
    const int* tile_expert;
    const int* tile_row0;
    const int* ntiles;
    const int* expert_offsets;
    const int* x_row;
    size_t expert_bytes;
    const uint8_t* w2;
    int n_split;
};
int mmq_group_rows(int rows_per_expert);  // tile height for an average rows-per-expert
hipError_t launch_mmq_grouped(int dtype, const uint8_t* w, ActView act, float* y, int bm, int max_tiles, int N, int K,
                              int ldy, const MmqGroup& g, hipStream_t s);
// Per-(m, n, block) integer sums, the bit-exact stage of the dot products.
hipError_t launch_block_isums(int dtype, const uint8_t* w, ActView act, int32_t* isum,
                              int32_t* msum, int M, int N, int K, hipStream_t s);

// dequant.hip: blocks -> f32 (or f16 bits) values, bit-exact with to_float.
hipError_t launch_dequantize(int dtype, const uint8_t* w, size_t nblocks, float* y16or32,
                             bool to_f16, hipStream_t s);

// weights.hip: from_float on the device (one thread per superblock), and the
// Philox synthetic-input generator.
hipError_t launch_quantize_weights(int dtype, const float* x, size_t nblocks, uint8_t* out, hipStream_t s);
// from_float_imatrix (Q4_K, Q6_K): superblock ib uses the importance weights
// imatrix[(ib % blocks_per_row) * 256 ...] (device memory).
hipError_t launch_quantize_weights_imatrix(int dtype, const float* x, size_t nblocks, const float* imatrix,
                                           size_t blocks_per_row, uint8_t* out, hipStream_t s);
hipError_t launch_random_bits(uint32_t* y, size_t n, unsigned long long start, unsigned long long seed,
                              uint32_t base, uint32_t stream, hipStream_t s);
hipError_t launch_normal(float* y, size_t n, unsigned long long seed, uint32_t stream, float mean, float stdv,
                         hipStream_t s);

// probe.hip: a read-only streaming kernel over `bytes` (a multiple of 16) with
// `grid` workgroups of 256 threads and `unroll` (1, 2, 4, 8) loads in flight
// per thread; the HBM read ceiling of a launch that size.
hipError_t launch_probe_read(const void* src, size_t bytes, int grid, int unroll, int nontemporal, uint32_t* sink,
                             hipStream_t s);

// decode.hip: attention of one new token per head over an f16 KV cache with
// RoPE and the cache append fused (head_dim ATTN_HEAD_DIM): a split kernel
// over context ranges writing (output, max, sum) partials to `part`
// (attn_decode_work_bytes), then a combine kernel; and the greedy next-token
// + embedding step.
constexpr int ATTN_HEAD_DIM = 128;
constexpr int ATTN_NIT = 4;                     // positions per 16-lane group and split
constexpr int ATTN_MAX_CHUNK = 32 * ATTN_NIT;   // positions per split (512-thread workgroups)
constexpr int ATTN_PSTRIDE = ATTN_HEAD_DIM + 4; // floats per (head, split) partial: o, max, sum, 2 pad (16-byte rows)
constexpr int ATTN_MERGE_CHUNK = 8;             // splits merged per step
int attn_decode_splits(int n_heads, int max_ctx);
size_t attn_decode_work_bytes(int n_heads, int max_ctx);
hipError_t launch_attn_decode(const float* qk, const float* v, const float* rcos, const float* rsin, uint16_t* kc,
                              uint16_t* vc, int n_heads, int max_ctx, const int* pos, float scale, float* part,
                              float* out, hipStream_t s);
// The split kernel alone (partials into `part`), for a consumer that merges
// them itself (launch_qmv_attn).
hipError_t launch_attn_split(const float* qk, const float* v, const float* rcos, const float* rsin, uint16_t* kc,
                             uint16_t* vc, int n_heads, int max_ctx, const int* pos, float scale, float* part,
                             hipStream_t s);
hipError_t launch_argmax_embed(const float* logits, int vocab, const float* table, int dim, int* tokens,
                               int tokens_cap, const int* prompt_len, int* pos, float* x, hipStream_t s);

// prefill.hip: row kernels of a batched prompt pass (M tokens at positions
// pos0 .. pos0 + M - 1) between the int8-MFMA projections.
hipError_t launch_rms_norm_rows(const float* x, int ldx, const float* gain, float eps, int M, int K, float* y, int ldy,
                                hipStream_t s);
hipError_t launch_rope_append_rows(float* qk, int ldqk, const float* v, int ldv, const float* rcos, const float* rsin,
                                   int M, int n_heads, int pos0, int max_ctx, uint16_t* kc, uint16_t* vc,
                                   hipStream_t s);
hipError_t launch_attention_prefill(const float* q, int ldq, const uint16_t* kc, const uint16_t* vc, int pos0, int M,
                                    int n_heads, int max_ctx, float scale, float* out, int ldo, hipStream_t s);
hipError_t launch_swiglu_rows(const float* gu, int ldgu, int M, int f, float* h, int ldh, hipStream_t s);
hipError_t launch_add_rows(const float* x, float* y, size_t n, hipStream_t s);
hipError_t launch_gather_rows(const float* table, int rows, int dim, const int* ids, int M, float* out,
                              hipStream_t s);

}  // namespace frq
