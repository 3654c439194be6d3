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

// mmvq.hip: y[m, n] = sum_b blockdot(W[n, b], act[m, b]) for rows m < M.
hipError_t launch_mmvq(int dtype, const uint8_t* w, ActView act, float* y, int M, int N, int K,
                       int ldy, hipStream_t s, int num_cus);
// Per-(m, n, block) integer sums, the bit-exact stage of the dot products.
hipError_t launch_block_isums(int dtype, const uint8_t* w, ActView act, int32_t* isum,
                              int32_t* msum, int M, int N, int K, hipStream_t s);

// dequant.hip: blocks -> f32 (or f16 bits) values, bit-exact with to_float.
hipError_t launch_dequantize(int dtype, const uint8_t* w, size_t nblocks, float* y16or32,
                             bool to_f16, hipStream_t s);

}  // namespace frq
