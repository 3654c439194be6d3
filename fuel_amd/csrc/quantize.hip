// Activation quantizers: f32 rows -> fuel's Q8K / Q8_0 int8 blocks, bit-exact
// with BlockQ8K::from_float (k_quants.rs:2230-2267) and BlockQ8_0::from_float
// (k_quants.rs:629-658).  Built with -ffp-contract=off; '/' is IEEE-correctly
// rounded (hipcc's default), roundf is half-away-from-zero like f32::round.
#include "common.hpp"
#include "kernels.hpp"

namespace frq {

// One wavefront per 256-element superblock; lane l holds elements 4l..4l+3.
// grid = (K/256, rows).  Writes the SoA workspace and, if aos != nullptr,
// fuel's BlockQ8K bytes.
__global__ __launch_bounds__(64) void quantize_q8k_kernel(const float* __restrict__ x, int K,
                                                          ActView act, uint8_t* __restrict__ aos) {
    const int b = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / QK_K;
    const float4 v = reinterpret_cast<const float4*>(x + (size_t)m * K + (size_t)b * QK_K)[lane];
    const float xv[4] = {v.x, v.y, v.z, v.w};

    // First element of largest |x| (strict '<' scan, so NaN and 0 never win).
    float best = 0.0f, bval = 0.0f;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float ax = fabsf(xv[i]);
        if (best < ax) {
            best = ax;
            bval = xv[i];
            bidx = 4 * lane + i;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ob = __shfl_xor(best, off, 64);
        const float ov = __shfl_xor(bval, off, 64);
        const int oi = __shfl_xor(bidx, off, 64);
        if (ob > best || (ob == best && oi < bidx)) {
            best = ob;
            bval = ov;
            bidx = oi;
        }
    }

    int q[4];
    float d;
    if (best == 0.0f) {
        q[0] = q[1] = q[2] = q[3] = 0;
        d = 0.0f;
    } else {
        const float iscale = -128.0f / bval;
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = sat_i8(fminf(roundf(iscale * xv[i]), 127.0f));
        d = 1.0f / iscale;
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);

    reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)b * QK_K)[lane] = packed;
    if ((lane & 3) == 0) act.bsums[((size_t)m * KB + b) * 16 + (lane >> 2)] = (int16_t)s;
    if (lane == 0) act.d[(size_t)m * KB + b] = d;
    if (aos) {
        uint8_t* blk = aos + ((size_t)m * KB + b) * Q8K_BYTES;
        reinterpret_cast<uint32_t*>(blk + 4)[lane] = packed;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(blk + 260)[lane >> 2] = (int16_t)s;
        if (lane == 0) *reinterpret_cast<float*>(blk) = d;
    }
}

// Eight 32-element blocks per wavefront; lane l holds elements 4l..4l+3 of
// block (l / 8).  grid = (ceil(K/256), rows).
__global__ __launch_bounds__(64) void quantize_q8_0_kernel(const float* __restrict__ x, int K,
                                                           ActView act, uint8_t* __restrict__ aos) {
    const int m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / QK8_0;
    const int blk = blockIdx.x * 8 + (lane >> 3);
    const bool live = blk < KB;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v = reinterpret_cast<const float4*>(x + (size_t)m * K + (size_t)blk * QK8_0)[lane & 7];
    const float xv[4] = {v.x, v.y, v.z, v.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(xv[i]));
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16_rne(d);
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = sat_i8(roundf(xv[i] * id));
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    if (!live) return;
    reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)blk * QK8_0)[lane & 7] = packed;
    if ((lane & 7) == 0) act.d[(size_t)m * KB + blk] = f16_to_f32(dh);
    if (aos) {
        uint8_t* p = aos + ((size_t)m * KB + blk) * Q8_0_BYTES;
        uint16_t* qs16 = reinterpret_cast<uint16_t*>(p + 2 + 4 * (lane & 7));
        qs16[0] = (uint16_t)(packed & 0xffffu);
        qs16[1] = (uint16_t)(packed >> 16);
        if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(p) = dh;
    }
}

hipError_t launch_quantize_q8k(const float* x, int rows, int K, ActView act, uint8_t* aos,
                               hipStream_t s) {
    dim3 grid(K / QK_K, rows);
    hipLaunchKernelGGL(quantize_q8k_kernel, grid, dim3(64), 0, s, x, K, act, aos);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float* x, int rows, int K, ActView act, uint8_t* aos,
                                hipStream_t s) {
    dim3 grid((K / QK8_0 + 7) / 8, rows);
    hipLaunchKernelGGL(quantize_q8_0_kernel, grid, dim3(64), 0, s, x, K, act, aos);
    return hipGetLastError();
}

}  // namespace frq
