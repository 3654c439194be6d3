// Row kernels of a batched prompt pass (prefill) through the LLaMA-shaped
// decoder: M tokens at positions pos0 .. pos0 + M - 1 go through every layer
// at once, with the int8-MFMA QMatMul (mmq.hip) for the projections and these
// kernels between them (fuel-core/src/lazy.rs:7363-7446 at seq = M):
//
//   rms_norm_rows     rms_norm_last_dim_f32 and the affine gain
//                     (byte_kernels.rs:2339-2368, lazy.rs:10330-10346) per row
//   rope_append_rows  rotate-half RoPE of q and k with the f32 tables
//                     (rope_f32, byte_kernels.rs:1885-1964), q in place, k and
//                     v rounded to f16 into the KV cache rows pos0 + m
//   attention_prefill causal scaled-dot-product attention of each query row
//                     over cache rows 0 .. its position (lazy.rs:7415-7425:
//                     scores * scale + causal mask, softmax_last_dim, . V),
//                     one pass with a running maximum, eight rows per step
//   swiglu_rows       silu(g) * u (lazy.rs:7442)
//   add_rows          the residual adds (lazy.rs:7434, 7446)
//   gather_rows       embedding rows of the prompt tokens
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "kernels.hpp"
#include "q8.hpp"

namespace frq {

namespace {

constexpr int HD = ATTN_HEAD_DIM;
constexpr int RN_WG = 256;

// y = (x * (1 / sqrt(sum(x^2) / K + eps))) * gain, one workgroup per row; the
// sum of squares is a tree over the workgroup (sequential in the reference).
__global__ __launch_bounds__(RN_WG) void rms_norm_rows_kernel(const float* __restrict__ x, int ldx,
                                                              const float* __restrict__ gain, float eps, int K,
                                                              float* __restrict__ y, int ldy) {
    __shared__ float s_red[RN_WG / 64];
    const int m = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (size_t)m * ldx;
    float ss = 0.0f;
    for (int i = tid; i < K; i += RN_WG) ss = fmaf(xr[i], xr[i], ss);
    ss = dpp_wave_sum(ss);
    if ((tid & 63) == 63) s_red[tid >> 6] = ss;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < RN_WG / 64; w++) total += s_red[w];
    const float rinv = 1.0f / sqrtf(total * (1.0f / (float)K) + eps);
    float* yr = y + (size_t)m * ldy;
    for (int i = tid; i < K; i += RN_WG) yr[i] = (xr[i] * rinv) * gain[i];
}

// grid (M, heads), HD threads: threads [0, HD/2) rotate q's pairs (i, i+HD/2)
// in place and append v's first half; threads [HD/2, HD) rotate k's pairs into
// the f16 cache and append v's second half.
__global__ __launch_bounds__(HD) void rope_append_rows_kernel(float* __restrict__ qk, int ldqk,
                                                              const float* __restrict__ v, int ldv,
                                                              const float* __restrict__ rcos,
                                                              const float* __restrict__ rsin, int pos0, int max_ctx,
                                                              __half* __restrict__ kc, __half* __restrict__ vc) {
    const int m = blockIdx.x, h = blockIdx.y, H = gridDim.y, tid = threadIdx.x;
    const int pos = pos0 + m;
    const float* cs = rcos + (size_t)pos * HD;
    const float* sn = rsin + (size_t)pos * HD;
    const int i = tid & (HD / 2 - 1);
    float* row = qk + (size_t)m * ldqk + (size_t)(tid < HD / 2 ? h : H + h) * HD;
    const float lo = row[i], hi = row[i + HD / 2];
    const float a = lo * cs[i] - hi * sn[i];
    const float b = hi * cs[i + HD / 2] + lo * sn[i + HD / 2];
    const size_t crow = ((size_t)h * max_ctx + pos) * HD;
    if (tid < HD / 2) {
        row[i] = a;
        row[i + HD / 2] = b;
    } else {
        kc[crow + i] = __float2half(a);
        kc[crow + i + HD / 2] = __float2half(b);
    }
    vc[crow + tid] = __float2half(v[(size_t)m * ldv + (size_t)h * HD + tid]);
}

constexpr int AP_WG = 256;
constexpr int AP_Q = AP_WG / 16;  // query rows per workgroup (16 lanes each, 8 dims per lane)
constexpr int AP_KB = 8;          // cache rows whose loads are in flight together

__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ void h8_to_f(const uint4& u, float (&f)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = __half2float(__ushort_as_half((unsigned short)(w[i] & 0xffffu)));
        f[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(w[i] >> 16)));
    }
}

// grid (heads, ceil(M / AP_Q)), AP_WG threads: 16-lane group g takes query row
// m = AP_Q * blockIdx.y + g (position pos0 + m) and walks cache rows
// 0 .. position AP_KB at a time with a running maximum: the step's scores
// s_j = (q . k_j) * scale, M' = max(M, s_j of the step), l = l e^(M - M') +
// sum e^(s_j - M'), o = o e^(M - M') + sum e^(s_j - M') v_j; out = o / l.
// Rows past a group's position (the wave runs to its last group's) are
// dropped by selects.
__global__ __launch_bounds__(AP_WG) void attention_prefill_kernel(const float* __restrict__ q, int ldq,
                                                                  const __half* __restrict__ kc,
                                                                  const __half* __restrict__ vc, int pos0, int M,
                                                                  int max_ctx, float scale, float* __restrict__ out,
                                                                  int ldo) {
    const int h = blockIdx.x, tid = threadIdx.x, g = tid >> 4, l16 = tid & 15;
    const int m = AP_Q * blockIdx.y + g;
    const int mq = m < M ? m : M - 1;
    const int pos = pos0 + mq;
    // the wave's last query row bounds its loop (4 groups per wave)
    const int wlast = min(AP_Q * (int)blockIdx.y + (tid >> 6) * 4 + 3, M - 1);
    const int jend = pos0 + wlast;
    const float* qr = q + (size_t)mq * ldq + (size_t)h * HD + 8 * l16;
    float q8[8];
#pragma unroll
    for (int e = 0; e < 8; e++) q8[e] = qr[e];
    const size_t cbase = (size_t)h * max_ctx * HD + 8 * l16;
    float mx = -__builtin_inff(), l = 0.0f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // AP_KB cache rows per step, all their loads issued before the first is
    // used (rows past jend repeat row jend and are skipped like any row past a
    // group's position), so a step costs one memory round trip, not AP_KB
    for (int j0 = 0; j0 <= jend; j0 += AP_KB) {
        uint4 kr[AP_KB], vr[AP_KB];
#pragma unroll
        for (int u = 0; u < AP_KB; u++) {
            const size_t jr = (size_t)min(j0 + u, jend) * HD;
            kr[u] = *reinterpret_cast<const uint4*>(kc + cbase + jr);
            vr[u] = *reinterpret_cast<const uint4*>(vc + cbase + jr);
        }
        // the step's scores (rows past the group's position: -inf), one
        // rescale to the step's maximum, then the rows' weighted values
        float sv[AP_KB];
        float mn = mx;
#pragma unroll
        for (int u = 0; u < AP_KB; u++) {
            float kv[8];
            h8_to_f(kr[u], kv);
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) d = fmaf(q8[e], kv[e], d);
            const float sc = group16_sum(d) * scale;
            sv[u] = j0 + u <= pos ? sc : -__builtin_inff();
            mn = fmaxf(mn, sv[u]);
        }
        const float c = expf(mx - mn);  // (the first step: mx = -inf, l = o = 0; row 0 is always live)
        l *= c;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] *= c;
#pragma unroll
        for (int u = 0; u < AP_KB; u++) {
            const bool live = j0 + u <= pos;
            const float p = expf(sv[u] - mn);
            float vv[8];
            h8_to_f(vr[u], vv);
            l = live ? l + p : l;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = live ? fmaf(p, vv[e], o[e]) : o[e];
        }
        mx = mn;
    }
    if (m < M) {
        float* orow = out + (size_t)m * ldo + (size_t)h * HD + 8 * l16;
#pragma unroll
        for (int e = 0; e < 8; e++) orow[e] = o[e] / l;
    }
}

__global__ void swiglu_rows_kernel(const float* __restrict__ gu, int ldgu, int f, float* __restrict__ h, int ldh) {
    const int m = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < f) h[(size_t)m * ldh + i] = silu_mul(gu[(size_t)m * ldgu + i], gu[(size_t)m * ldgu + f + i]);
}

__global__ void add_rows_kernel(const float* __restrict__ x, float* __restrict__ y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] += x[i];
}

__global__ void gather_rows_kernel(const float* __restrict__ table, int rows, int dim, const int* __restrict__ ids,
                                   float* __restrict__ out) {
    const int m = blockIdx.y;
    int id = ids[m];
    if ((unsigned)id >= (unsigned)rows) id = 0;  // an out-of-range id reads row 0 (as argmax_embed)
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x)
        out[(size_t)m * dim + i] = table[(size_t)id * dim + i];
}

}  // namespace

hipError_t launch_rms_norm_rows(const float* x, int ldx, const float* gain, float eps, int M, int K, float* y, int ldy,
                                hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_rows_kernel, dim3(M), dim3(RN_WG), 0, s, x, ldx, gain, eps, K, y, ldy);
    return hipGetLastError();
}

hipError_t launch_rope_append_rows(float* qk, int ldqk, const float* v, int ldv, const float* rcos, const float* rsin,
                                   int M, int n_heads, int pos0, int max_ctx, uint16_t* kc, uint16_t* vc,
                                   hipStream_t s) {
    hipLaunchKernelGGL(rope_append_rows_kernel, dim3(M, n_heads), dim3(HD), 0, s, qk, ldqk, v, ldv, rcos, rsin, pos0,
                       max_ctx, reinterpret_cast<__half*>(kc), reinterpret_cast<__half*>(vc));
    return hipGetLastError();
}

hipError_t launch_attention_prefill(const float* q, int ldq, const uint16_t* kc, const uint16_t* vc, int pos0, int M,
                                    int n_heads, int max_ctx, float scale, float* out, int ldo, hipStream_t s) {
    hipLaunchKernelGGL(attention_prefill_kernel, dim3(n_heads, (M + AP_Q - 1) / AP_Q), dim3(AP_WG), 0, s, q, ldq,
                       reinterpret_cast<const __half*>(kc), reinterpret_cast<const __half*>(vc), pos0, M, max_ctx,
                       scale, out, ldo);
    return hipGetLastError();
}

hipError_t launch_swiglu_rows(const float* gu, int ldgu, int M, int f, float* h, int ldh, hipStream_t s) {
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((f + 255) / 256, M), dim3(256), 0, s, gu, ldgu, f, h, ldh);
    return hipGetLastError();
}

hipError_t launch_add_rows(const float* x, float* y, size_t n, hipStream_t s) {
    hipLaunchKernelGGL(add_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float* table, int rows, int dim, const int* ids, int M, float* out,
                              hipStream_t s) {
    const int bx = (dim + 255) / 256 < 16 ? (dim + 255) / 256 : 16;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(bx, M), dim3(256), 0, s, table, rows, dim, ids, out);
    return hipGetLastError();
}

}  // namespace frq
