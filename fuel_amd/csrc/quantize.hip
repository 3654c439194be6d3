// Standalone activation quantizers (f32 rows -> fuel's Q8K / Q8_0 blocks), used
// by the integer taps and the batched path; the arithmetic is q8.hpp's.
#include "common.hpp"
#include "kernels.hpp"
#include "q8.hpp"

namespace frq {

// One wavefront per 256-element superblock; grid = (K/256, rows).  Writes the
// SoA workspace and, if aos != nullptr, fuel's BlockQ8K bytes.
__global__ __launch_bounds__(64) void quantize_q8k_kernel(const float* __restrict__ x, int ldx, int K,
                                                          ActView act, uint8_t* __restrict__ aos) {
    const int b = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / QK_K;
    const Q8KWave r = q8k_quantize_wave(x + (size_t)m * ldx + (size_t)b * QK_K, lane);
    reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)b * QK_K)[lane] = r.packed;
    if ((lane & 3) == 0) {
        act.bsums[((size_t)m * KB + b) * 16 + (lane >> 2)] = (int16_t)r.bsum;
        if (act.bsh) act.bsh[((size_t)m * KB + b) * 16 + (lane >> 2)] = f32_to_f16_rne((float)r.bsum);
    }
    if (lane == 0) act.d[(size_t)m * KB + b] = r.d;
    if (aos) {
        uint8_t* blk = aos + ((size_t)m * KB + b) * Q8K_BYTES;
        reinterpret_cast<uint32_t*>(blk + 4)[lane] = r.packed;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(blk + 260)[lane >> 2] = (int16_t)r.bsum;
        if (lane == 0) *reinterpret_cast<float*>(blk) = r.d;
    }
}

// f16 rows (matmul_f16): each half widened exactly to f32, then the same
// from_float as above; grid = (K/256, rows).
__global__ __launch_bounds__(64) void quantize_q8k_h_kernel(const uint16_t* __restrict__ x, int K, ActView act) {
    const int b = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / QK_K;
    const uint2 h = reinterpret_cast<const uint2*>(x + (size_t)m * K + (size_t)b * QK_K)[lane];
    const float4 v = make_float4(f16_to_f32(h.x & 0xffffu), f16_to_f32(h.x >> 16), f16_to_f32(h.y & 0xffffu),
                                 f16_to_f32(h.y >> 16));
    const Q8KWave r = q8k_quantize_vals(v, lane);
    reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)b * QK_K)[lane] = r.packed;
    if ((lane & 3) == 0) {
        act.bsums[((size_t)m * KB + b) * 16 + (lane >> 2)] = (int16_t)r.bsum;
        if (act.bsh) act.bsh[((size_t)m * KB + b) * 16 + (lane >> 2)] = f32_to_f16_rne((float)r.bsum);
    }
    if (lane == 0) act.d[(size_t)m * KB + b] = r.d;
}

// SwiGLU input of the down projection: rows of silu(g) * u, g rows in x and
// u rows in x2 (both of row stride ldx); grid = (K/256, rows).
__global__ __launch_bounds__(64) void quantize_q8k_swiglu_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ x2, int ldx, int K,
                                                                 ActView act) {
    const int b = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / QK_K;
    const size_t o = (size_t)m * ldx + (size_t)b * QK_K;
    const float4 gv = reinterpret_cast<const float4*>(x + o)[lane];
    const float4 uv = reinterpret_cast<const float4*>(x2 + o)[lane];
    const float4 h = make_float4(silu_mul(gv.x, uv.x), silu_mul(gv.y, uv.y), silu_mul(gv.z, uv.z),
                                 silu_mul(gv.w, uv.w));
    const Q8KWave r = q8k_quantize_vals(h, lane);
    reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)b * QK_K)[lane] = r.packed;
    if ((lane & 3) == 0) {
        act.bsums[((size_t)m * KB + b) * 16 + (lane >> 2)] = (int16_t)r.bsum;
        if (act.bsh) act.bsh[((size_t)m * KB + b) * 16 + (lane >> 2)] = f32_to_f16_rne((float)r.bsum);
    }
    if (lane == 0) act.d[(size_t)m * KB + b] = r.d;
}

// Rows of rms_norm(x) * gain quantized to Q8K: one workgroup of QR_NW
// wavefronts per row, the row held in registers (wavefront w owns chunks w,
// w + QR_NW, ...); the norm is the fused mat-vec prologue's arithmetic
// (q8.hpp act_row_rms_norm: per-lane sums of squares, DPP wave sums, the
// wavefronts' sums added in order).  grid = rows.
constexpr int QR_NW = 16;

template <int MAXQ>
__global__ __launch_bounds__(64 * QR_NW) void quantize_q8k_rms_kernel(const float* __restrict__ x, int ldx,
                                                                      const float* __restrict__ gain, float eps,
                                                                      int K, ActView act) {
    __shared__ float s_red[QR_NW];
    const int m = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int KB = K / QK_K;
    ActRowPre<MAXQ> pre;
    act_row_load<GGML_Q8K, QR_NW, MAXQ>(x + (size_t)m * ldx, K, w, lane, pre);
    act_row_rms_norm<GGML_Q8K, QR_NW, MAXQ>(pre, gain, eps, K, w, lane, [&](float v) {
        if (lane == 63) s_red[w] = v;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < QR_NW; i++) t += s_red[i];
        return t;
    });
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {
        const int b = w + QR_NW * i;
        if (b >= KB) break;
        const Q8KWave r = q8k_quantize_vals(pre.v[i], lane);
        reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)b * QK_K)[lane] = r.packed;
        if ((lane & 3) == 0) {
            act.bsums[((size_t)m * KB + b) * 16 + (lane >> 2)] = (int16_t)r.bsum;
            if (act.bsh) act.bsh[((size_t)m * KB + b) * 16 + (lane >> 2)] = f32_to_f16_rne((float)r.bsum);
        }
        if (lane == 0) act.d[(size_t)m * KB + b] = r.d;
    }
}

// Eight 32-element blocks per wavefront; grid = (ceil(K/256), rows).
__global__ __launch_bounds__(64) void quantize_q8_0_kernel(const float* __restrict__ x, int K,
                                                           ActView act, uint8_t* __restrict__ aos) {
    const int m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / QK8_0;
    const int blk = blockIdx.x * 8 + (lane >> 3);
    const bool live = blk < KB;
    const Q80Wave r = q8_0_quantize_wave(x + (size_t)m * K + (size_t)blk * QK8_0, live, lane);
    if (!live) return;
    reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)blk * QK8_0)[lane & 7] = r.packed;
    if ((lane & 7) == 0) act.d[(size_t)m * KB + blk] = f16_to_f32(r.dbits);
    if (aos) {
        uint8_t* p = aos + ((size_t)m * KB + blk) * Q8_0_BYTES;
        uint16_t* qs16 = reinterpret_cast<uint16_t*>(p + 2 + 4 * (lane & 7));
        qs16[0] = (uint16_t)(r.packed & 0xffffu);
        qs16[1] = (uint16_t)(r.packed >> 16);
        if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(p) = r.dbits;
    }
}

// f16 rows of the Q8_0 path (matmul_f16): halves widened exactly to f32, then
// the Q8_0 from_float of the kernel above; grid = (ceil(K/256), rows).
__global__ __launch_bounds__(64) void quantize_q8_0_h_kernel(const uint16_t* __restrict__ x, int K, ActView act) {
    const int m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / QK8_0;
    const int blk = blockIdx.x * 8 + (lane >> 3);
    const bool live = blk < KB;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
        const uint2 h = reinterpret_cast<const uint2*>(x + (size_t)m * K + (size_t)blk * QK8_0)[lane & 7];
        v = make_float4(f16_to_f32(h.x & 0xffffu), f16_to_f32(h.x >> 16), f16_to_f32(h.y & 0xffffu),
                        f16_to_f32(h.y >> 16));
    }
    const Q80Wave r = q8_0_quantize_vals(v, lane);
    if (!live) return;
    reinterpret_cast<uint32_t*>(act.qs + (size_t)m * K + (size_t)blk * QK8_0)[lane & 7] = r.packed;
    if ((lane & 7) == 0) act.d[(size_t)m * KB + blk] = f16_to_f32(r.dbits);
}

hipError_t launch_quantize_q8_0_h(const uint16_t* x, int rows, int K, ActView act, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_0_h_kernel, dim3((K / QK8_0 + 7) / 8, rows), dim3(64), 0, s, x, K, act);
    return hipGetLastError();
}

hipError_t launch_quantize_q8k(const float* x, int rows, int K, ActView act, uint8_t* aos,
                               hipStream_t s) {
    dim3 grid(K / QK_K, rows);
    hipLaunchKernelGGL(quantize_q8k_kernel, grid, dim3(64), 0, s, x, K, K, act, aos);
    return hipGetLastError();
}

hipError_t launch_quantize_q8k_h(const uint16_t* x, int rows, int K, ActView act, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8k_h_kernel, dim3(K / QK_K, rows), dim3(64), 0, s, x, K, act);
    return hipGetLastError();
}

hipError_t launch_quantize_q8k_swiglu(const float* x, int ldx, int rows, int K, ActView act, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8k_swiglu_kernel, dim3(K / QK_K, rows), dim3(64), 0, s, x, x + K, ldx, K, act);
    return hipGetLastError();
}

bool quantize_src_supported(const ActSrc& src, int K) {
    return K % QK_K == 0 && !(src.x2 && src.gain) && (!src.gain || K <= 8 * QR_NW * QK_K);
}

hipError_t launch_quantize_q8k_src(const ActSrc& src, int rows, int K, ActView act, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (!quantize_src_supported(src, K)) return hipErrorInvalidValue;
    if (src.x2) {
        hipLaunchKernelGGL(quantize_q8k_swiglu_kernel, dim3(K / QK_K, rows), dim3(64), 0, s, src.x, src.x2, src.ldx,
                           K, act);
    } else if (src.gain) {
        const int maxq = (K / QK_K + QR_NW - 1) / QR_NW;
#define FRQ_QR(q)                                                                                                 \
    case q:                                                                                                       \
        hipLaunchKernelGGL(quantize_q8k_rms_kernel<q>, dim3(rows), dim3(64 * QR_NW), 0, s, src.x, src.ldx, src.gain, \
                           src.eps, K, act);                                                                      \
        break;
        switch (maxq) {
            FRQ_QR(1) FRQ_QR(2) FRQ_QR(3) FRQ_QR(4) FRQ_QR(5) FRQ_QR(6) FRQ_QR(7) FRQ_QR(8)
            default: return hipErrorInvalidValue;
        }
#undef FRQ_QR
    } else {
        hipLaunchKernelGGL(quantize_q8k_kernel, dim3(K / QK_K, rows), dim3(64), 0, s, src.x, src.ldx, K, act,
                           (uint8_t*)nullptr);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float* x, int rows, int K, ActView act, uint8_t* aos,
                                hipStream_t s) {
    dim3 grid((K / QK8_0 + 7) / 8, rows);
    hipLaunchKernelGGL(quantize_q8_0_kernel, grid, dim3(64), 0, s, x, K, act, aos);
    return hipGetLastError();
}

}  // namespace frq
