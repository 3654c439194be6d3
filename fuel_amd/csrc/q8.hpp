// Wave-level activation quantizers, bit-exact with BlockQ8K::from_float
// (k_quants.rs:2230-2267) and BlockQ8_0::from_float (k_quants.rs:629-658).
// One definition serves the standalone quantize kernels and the fused
// quantize+mat-vec kernels.  Translation units including this header are
// built with -ffp-contract=off: nothing here may fuse into an FMA.
#pragma once

#include "common.hpp"

namespace frq {

// Quantized values of one 256-element superblock held by a wavefront: lane l
// owns elements 4l..4l+3 (packed int8 in `packed`), `bsum` is the sum of its
// 16-element group (valid in every lane of the group), `d` the block scale.
struct Q8KWave {
    uint32_t packed;
    int bsum;
    float d;
};

__device__ __forceinline__ Q8KWave q8k_quantize_wave(const float* __restrict__ x256, int lane) {
    const float4 v = reinterpret_cast<const float4*>(x256)[lane];
    const float xv[4] = {v.x, v.y, v.z, v.w};
    // First element of largest |x| (strict '<' scan: NaN and 0 never win).
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
    Q8KWave r;
    r.packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
               ((uint32_t)(q[3] & 0xff) << 24);
    r.bsum = s;
    r.d = d;
    return r;
}

// Eight 32-element blocks per wavefront: lane l owns elements 4(l%8).. of
// block l/8.  `live` lanes hold a real block.
struct Q80Wave {
    uint32_t packed;
    uint16_t dbits;
};

__device__ __forceinline__ Q80Wave q8_0_quantize_wave(const float* __restrict__ x32, bool live, int lane) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v = reinterpret_cast<const float4*>(x32)[lane & 7];
    const float xv[4] = {v.x, v.y, v.z, v.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(xv[i]));
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = sat_i8(roundf(xv[i] * id));
    Q80Wave r;
    r.packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
               ((uint32_t)(q[3] & 0xff) << 24);
    r.dbits = f32_to_f16_rne(d);
    return r;
}

// Quantize one activation row x[K] into an ActView row (qs / d / bsums), with
// the wavefronts w = 0..nw-1 of a workgroup sharing the blocks.
__device__ __forceinline__ void q8k_quantize_row(const float* __restrict__ x, int K, int8_t* qs, float* dv,
                                                 int16_t* bsums, int w, int nw, int lane) {
    const int KB = K / QK_K;
    for (int b = w; b < KB; b += nw) {
        const Q8KWave r = q8k_quantize_wave(x + (size_t)b * QK_K, lane);
        reinterpret_cast<uint32_t*>(qs + (size_t)b * QK_K)[lane] = r.packed;
        if ((lane & 3) == 0) bsums[b * 16 + (lane >> 2)] = (int16_t)r.bsum;
        if (lane == 0) dv[b] = r.d;
    }
}

__device__ __forceinline__ void q8_0_quantize_row(const float* __restrict__ x, int K, int8_t* qs, float* dv,
                                                  int w, int nw, int lane) {
    const int KB = K / QK8_0;
    for (int c = w; c * 8 < KB; c += nw) {
        const int blk = c * 8 + (lane >> 3);
        const bool live = blk < KB;
        const Q80Wave r = q8_0_quantize_wave(x + (size_t)blk * QK8_0, live, lane);
        if (live) {
            reinterpret_cast<uint32_t*>(qs + (size_t)blk * QK8_0)[lane & 7] = r.packed;
            if ((lane & 7) == 0) dv[blk] = f16_to_f32(r.dbits);
        }
    }
}

}  // namespace frq
