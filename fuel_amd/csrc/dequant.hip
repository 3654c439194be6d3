// Dequantize blocks to f32 (DynQuantizedStorage::dequantize) or f16
// (dequantize_f16), bit-exact with to_float: Q8_0 k_quants.rs:611-627,
// Q4K :1595-1622, Q6K :2158-2189.  Built with -ffp-contract=off so
// d1*q - m1 rounds twice, as in the reference.
#include "common.hpp"
#include "kernels.hpp"

namespace frq {

template <bool F16>
__device__ __forceinline__ void store4(void* y, size_t idx, float a, float b, float c, float d) {
    if constexpr (F16) {
        uint2 v;
        v.x = (uint32_t)f32_to_f16_rne(a) | ((uint32_t)f32_to_f16_rne(b) << 16);
        v.y = (uint32_t)f32_to_f16_rne(c) | ((uint32_t)f32_to_f16_rne(d) << 16);
        reinterpret_cast<uint2*>(y)[idx / 4] = v;
    } else {
        reinterpret_cast<float4*>(y)[idx / 4] = make_float4(a, b, c, d);
    }
}

// One wavefront per superblock; lane l writes elements 4l..4l+3.
template <bool F16>
__global__ __launch_bounds__(64) void dequant_q4k_kernel(const uint8_t* __restrict__ w, void* y) {
    const size_t ib = blockIdx.x;
    const int lane = threadIdx.x;
    const uint8_t* blk = w + ib * Q4K_BYTES;
    const int e = 4 * lane;                 // element within the superblock
    const int c = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    const int j = 2 * c + hi;               // sub-block
    const uint8_t* sc = blk + 4;
    int s, m;
    if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
    } else {
        s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    const float d = f16_to_f32(load_u16(blk)), dmin = f16_to_f32(load_u16(blk + 2));
    const float d1 = d * (float)s, m1 = dmin * (float)m;
    const uint32_t q = *reinterpret_cast<const uint32_t*>(blk + 16 + 32 * c + l);
    const uint32_t n = hi ? ((q >> 4) & 0x0f0f0f0fu) : (q & 0x0f0f0f0fu);
    store4<F16>(y, ib * QK_K + e, d1 * (float)(n & 0xff) - m1, d1 * (float)((n >> 8) & 0xff) - m1,
                d1 * (float)((n >> 16) & 0xff) - m1, d1 * (float)(n >> 24) - m1);
}

template <bool F16>
__global__ __launch_bounds__(64) void dequant_q6k_kernel(const uint8_t* __restrict__ w, void* y) {
    const size_t ib = blockIdx.x;
    const int lane = threadIdx.x;
    const uint8_t* blk = w + ib * Q6K_BYTES;
    const int e = 4 * lane;
    const int hh = e >> 7, r = e & 127, qd = r >> 5, l = r & 31;
    const float d = f16_to_f32(load_u16(blk + 208));
    const int8_t scv = (int8_t)blk[192 + 8 * hh + (l >> 4) + 2 * qd];
    const uint8_t* ql = blk + 64 * hh + 32 * (qd & 1) + l;
    const uint8_t* qh = blk + 128 + 32 * hh + l;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int lo = (qd >> 1) ? (ql[i] >> 4) : (ql[i] & 0xF);
        const int hb = (qh[i] >> (2 * qd)) & 3;
        const int q = (lo | (hb << 4)) - 32;
        v[i] = d * (float)scv * (float)q;
    }
    store4<F16>(y, ib * QK_K + e, v[0], v[1], v[2], v[3]);
}

// Eight 32-element blocks per wavefront.
template <bool F16>
__global__ __launch_bounds__(64) void dequant_q8_0_kernel(const uint8_t* __restrict__ w, size_t nblocks,
                                                          void* y) {
    const size_t ib = (size_t)blockIdx.x * 8 + (threadIdx.x >> 3);
    if (ib >= nblocks) return;
    const int t = threadIdx.x & 7;
    const uint8_t* blk = w + ib * Q8_0_BYTES;
    const float d = f16_to_f32(load_u16(blk));
    const int8_t* qs = reinterpret_cast<const int8_t*>(blk + 2 + 4 * t);
    store4<F16>(y, ib * QK8_0 + 4 * t, (float)qs[0] * d, (float)qs[1] * d, (float)qs[2] * d,
                (float)qs[3] * d);
}

hipError_t launch_dequantize(int dtype, const uint8_t* w, size_t nblocks, float* y, bool to_f16,
                             hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    switch (dtype) {
        case GGML_Q4K:
            if (to_f16) hipLaunchKernelGGL(dequant_q4k_kernel<true>, dim3(nblocks), dim3(64), 0, s, w, (void*)y);
            else hipLaunchKernelGGL(dequant_q4k_kernel<false>, dim3(nblocks), dim3(64), 0, s, w, (void*)y);
            break;
        case GGML_Q6K:
            if (to_f16) hipLaunchKernelGGL(dequant_q6k_kernel<true>, dim3(nblocks), dim3(64), 0, s, w, (void*)y);
            else hipLaunchKernelGGL(dequant_q6k_kernel<false>, dim3(nblocks), dim3(64), 0, s, w, (void*)y);
            break;
        case GGML_Q8_0: {
            dim3 grid((unsigned)((nblocks + 7) / 8));
            if (to_f16) hipLaunchKernelGGL(dequant_q8_0_kernel<true>, grid, dim3(64), 0, s, w, nblocks, (void*)y);
            else hipLaunchKernelGGL(dequant_q8_0_kernel<false>, grid, dim3(64), 0, s, w, nblocks, (void*)y);
            break;
        }
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace frq
