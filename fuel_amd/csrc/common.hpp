// Shared device helpers for the gfx950 quantized-matmul kernels.
//
// Block formats are the GGUF ones fuel uses (fuel-quantized/src/k_quants.rs
// :92-169): BlockQ8_0 34 B, BlockQ4K 144 B, BlockQ6K 210 B, BlockQ8K 292 B.
// Weights stay in that byte layout in HBM (row-major [N, K/blk] blocks), so a
// buffer produced by fuel's quantizer or read from a GGUF file is usable as is.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frq {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int Q8_0_BYTES = 34;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8K_BYTES = 292;

// GgmlDType codes (fuel-ir/src/quantized.rs:36-76).
enum : int { GGML_F32 = 0, GGML_F16 = 1, GGML_Q8_0 = 8, GGML_Q4K = 12, GGML_Q6K = 14, GGML_Q8K = 15 };

__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// IEEE binary16 round-to-nearest-even, written on integers so the result does
// not depend on the MODE register; same conversion as `half::f16::from_f32`.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? (0x0200u | (man >> 13)) : 0u));
    int e = (int)exp - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t sig = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t q = sig >> shift;
        uint32_t rem = sig & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

// Output modes of the matmul epilogues (the `out_mode` kernel argument):
// OUT_F16 stores f16 outputs (f16::from_f32 of the f32 sum), OUT_ACC adds
// the sum to the f32 output already in y (the residual add of a layer:
// y + v, fuel's x + proj order), neither stores the f32 sum.
constexpr int OUT_F16 = 1, OUT_ACC = 2;
__device__ __forceinline__ void store_out(float* y, size_t i, float v, int out_mode) {
    if (out_mode & OUT_F16) reinterpret_cast<uint16_t*>(y)[i] = f32_to_f16_rne(v);
    else if (out_mode & OUT_ACC) y[i] = y[i] + v;
    else y[i] = v;
}

// Rust `f as i8`: saturating, NaN -> 0.
__device__ __forceinline__ int sat_i8(float v) {
    if (v != v) return 0;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int)v;
}

// Rust `v.round() as i32` (utils.rs:1-3): half away from zero, saturating.
__device__ __forceinline__ int nearest_int(float v) {
    float r = roundf(v);
    if (r != r) return 0;
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return (int)0x80000000;
    return (int)r;
}

// 16 / 8 bytes at any byte address as one global load.  gfx950 under the HSA
// ABI runs with unaligned global access enabled (the compiler itself emits
// global_load_dwordx4 for an unaligned memcpy); the load reads exactly the
// requested bytes.
__device__ __forceinline__ uint4 load16_u(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

__device__ __forceinline__ uint2 load8_u(const uint8_t* p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}

__device__ __forceinline__ uint32_t load_u16(const uint8_t* p) {
    return (uint32_t)*(const uint16_t*)p;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Sum over the 64 lanes of a wavefront; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Wave64 sum through DPP row operations; the total is valid in lane 63 only.
__device__ __forceinline__ float dpp_wave_sum(float v) {
#define FRQ_DPP_ADD(ctrl, rmask)                                                                         \
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rmask, \
                                                               0xF, false))
    FRQ_DPP_ADD(0xB1, 0xF);   // quad_perm [1,0,3,2]
    FRQ_DPP_ADD(0x4E, 0xF);   // quad_perm [2,3,0,1]
    FRQ_DPP_ADD(0x141, 0xF);  // row_half_mirror: each 8-lane half holds its sum
    FRQ_DPP_ADD(0x140, 0xF);  // row_mirror: each 16-lane row holds its sum
    FRQ_DPP_ADD(0x142, 0xA);  // row_bcast:15 -> rows 1, 3 add rows 0, 2
    FRQ_DPP_ADD(0x143, 0xC);  // row_bcast:31 -> row 3 adds rows 0+1
#undef FRQ_DPP_ADD
    return v;
}

// Sum over each 64/RPW-lane segment of the wavefront (RPW = 2 or 4), in the
// order dpp_wave_sum adds those lanes; valid in the segment's last lane (with
// RPW = 4 in every lane of the 16-lane segment).
template <int RPW>
__device__ __forceinline__ float dpp_seg_sum(float v) {
    static_assert(RPW == 2 || RPW == 4, "segments of 32 or 16 lanes");
#define FRQ_DPP_ADD(ctrl, rmask)                                                                         \
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rmask, \
                                                               0xF, false))
    FRQ_DPP_ADD(0xB1, 0xF);
    FRQ_DPP_ADD(0x4E, 0xF);
    FRQ_DPP_ADD(0x141, 0xF);
    FRQ_DPP_ADD(0x140, 0xF);  // each 16-lane row holds its sum
    if constexpr (RPW == 2) FRQ_DPP_ADD(0x142, 0xA);  // rows 1, 3 add rows 0, 2
#undef FRQ_DPP_ADD
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Activation workspace.  The mat-vec kernels read activations as int8 quants
// in a structure-of-arrays layout (16-byte aligned rows); the byte layout of
// fuel's BlockQ8K / BlockQ8_0 is produced on request by the tap kernels.
//   qs    : int8  [rows][K]
//   d     : f32   [rows][K/blk]    (Q8K: the f32 d; Q8_0: f16 d widened)
//   bsums : int16 [rows][K/256][16] (Q8K only: sums of 16 consecutive quants)
//   bsh   : f16   [rows][K/256][16] (Q8K only: the same sums as binary16 bits,
//           exact since |sum| <= 2032; an MFMA operand of the batched kernel)
// ---------------------------------------------------------------------------
struct ActView {
    int8_t* qs;
    float* d;
    int16_t* bsums;
    uint16_t* bsh;
};

// LDS copy of one quantized activation row inside the mat-vec kernels.  Q8K
// superblocks sit 272 bytes apart (256 + 16 of padding) so the 16 lane groups
// of a wavefront, which read the same offset of 16 different superblocks, hit
// different LDS banks; each section starts 16-byte aligned.
struct ActLds {
    int qstride;   // bytes between consecutive activation blocks
    int off_d;     // f32 scales
    int off_bs;    // int16 bsums (Q8K)
    int bytes;     // total
};

__host__ __device__ constexpr int align16i(int x) { return (x + 15) & ~15; }

// qstride: bytes between the superblocks of a Q8K row in LDS (0: 256 + 16);
// the weight format picks the stride its lanes' reads are bank-conflict free
// with (formats.hpp, QSTRIDE).
__host__ __device__ inline ActLds act_lds_layout(int act_dtype, int K, int qstride = 0) {
    ActLds l{};
    if (act_dtype == GGML_Q8K) {
        const int kb = K / QK_K;
        l.qstride = qstride ? qstride : QK_K + 16;
        l.off_d = align16i(kb * l.qstride);
        l.off_bs = align16i(l.off_d + 4 * kb);
        l.bytes = l.off_bs + 32 * kb;
    } else {
        const int kb = K / QK8_0;
        l.qstride = QK8_0;
        l.off_d = align16i(K);
        l.off_bs = align16i(l.off_d + 4 * kb);
        l.bytes = l.off_bs;
    }
    return l;
}

// First-index argmax of fuel's scans (argextremum_dim_f32, fuel-cpu-backend/
// src/byte_kernels.rs:8178-8241: element 0 is taken unconditionally, then
// element d replaces the best when v > best) as a max under a total order, so
// that any reduction tree gives the scan's answer: larger key wins, equal keys
// go to the lower index, and scan_key maps a NaN at index 0 to +inf (never
// displaced) and any other NaN to -inf (never taken).
__device__ __forceinline__ float scan_key(float v, int j) {
    return v != v ? (j == 0 ? __builtin_inff() : -__builtin_inff()) : v;
}

// (bitwise and selects: no branch or exec-mask juggling in the reductions)
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    const bool take = (ov > v) | ((ov == v) & (oi < i));
    v = take ? ov : v;
    i = take ? oi : i;
}

// Wave64 reduction of (key, index) pairs under argmax_merge's total order
// (any tree gives the same pair): DPP row steps leave each 16-lane row's best
// in its lanes, four readlanes combine the rows.  The result is wave-uniform.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#define FRQ_DPP_ARGMAX(ctrl)                                                                                     \
    {                                                                                                           \
        const float ov =                                                                                        \
            __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false)); \
        const int oi = __builtin_amdgcn_update_dpp(0, i, ctrl, 0xF, 0xF, false);                                 \
        argmax_merge(v, i, ov, oi);                                                                             \
    }
    FRQ_DPP_ARGMAX(0xB1);   // quad_perm [1,0,3,2]
    FRQ_DPP_ARGMAX(0x4E);   // quad_perm [2,3,0,1]
    FRQ_DPP_ARGMAX(0x141);  // row_half_mirror
    FRQ_DPP_ARGMAX(0x140);  // row_mirror
#undef FRQ_DPP_ARGMAX
    float bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16)
        argmax_merge(bv, bi, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), r)),
                     __builtin_amdgcn_readlane(i, r));
    v = bv;
    i = bi;
}

}  // namespace frq
