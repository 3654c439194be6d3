// Host-side launchers of the device kernels (one translation unit each).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace frq {

// quantize.hip
hipError_t launch_quantize_q8k(const float* x, int rows, int K, ActView act, uint8_t* aos,
                               hipStream_t s);
hipError_t launch_quantize_q8_0(const float* x, int rows, int K, ActView act, uint8_t* aos,
                                hipStream_t s);

// mmvq.hip: y[m, n] = sum_b blockdot(W[n, b], quantize(x[m])_b) for rows m < M,
// activation quantization fused into the kernel.
hipError_t launch_qmv(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K,
                      int ldy, hipStream_t s, int num_cus);
// mmq.hip: int8-MFMA matmul for M >= 16 over activations already quantized
// into the workspace (quantize_q8k), y [M, N] with row stride ldy.
// `part` (part_elems floats, may be null) holds split-K partial sums.
bool mmq_supported(int dtype);
size_t mmq_partial_elems(int M, int N, int num_cus);
hipError_t launch_mmq(int dtype, const uint8_t* w, ActView act, float* y, float* part, size_t part_elems, int M,
                      int N, int K, int ldy, int num_cus, hipStream_t s);
// Per-(m, n, block) integer sums, the bit-exact stage of the dot products.
hipError_t launch_block_isums(int dtype, const uint8_t* w, ActView act, int32_t* isum,
                              int32_t* msum, int M, int N, int K, hipStream_t s);

// dequant.hip: blocks -> f32 (or f16 bits) values, bit-exact with to_float.
hipError_t launch_dequantize(int dtype, const uint8_t* w, size_t nblocks, float* y16or32,
                             bool to_f16, hipStream_t s);

// weights.hip: from_float on the device (one thread per superblock), and the
// Philox synthetic-input generator.
hipError_t launch_quantize_weights(int dtype, const float* x, size_t nblocks, uint8_t* out, hipStream_t s);
hipError_t launch_random_bits(uint32_t* y, size_t n, unsigned long long start, unsigned long long seed,
                              uint32_t base, uint32_t stream, hipStream_t s);
hipError_t launch_normal(float* y, size_t n, unsigned long long seed, uint32_t stream, float mean, float stdv,
                         hipStream_t s);

}  // namespace frq
