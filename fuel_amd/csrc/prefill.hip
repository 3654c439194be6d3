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
//                     one pass with a running maximum, on f16 MFMA with the
//                     f32 operands split exactly into two f16 halves
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

// Attention of a query tile on f16 MFMA.  A workgroup owns 16 query rows of
// one head; its AF_WAVES wavefronts split the tile's cache rows 0 .. its last
// row's position into contiguous ranges of 16-row blocks, and each walks its
// range with a running maximum (flash attention):
//   S^T (16 keys x 16 queries) = K_blk (16 x 128) . Q^T (128 x 16) on
//     v_mfma_f32_16x16x32_f16, four 32-dim steps; K rows are f16 already and
//     each q value is split exactly into f16 hi + lo (hi = f16(q), lo =
//     f16(q - hi): hi + lo = q to 2^-22), two MFMAs per step, f32 sums;
//   s = S^T * scale, causal mask by select, block max / sum over the 16 keys,
//     rescale of the running sum and output;
//   O^T (128 x 16) += V^T (128 x 16 keys) . P^T (16 keys x 16) on
//     v_mfma_f32_16x16x16_f16 per 16-dim tile, P split into f16 hi + lo the
//     same way.
// Lane l = 16 g + r: the S^T MFMA's C layout leaves it keys 4g + i (i < 4) of
// query r, which is exactly the B operand (keys 4g .. 4g+3, column r) the PV
// MFMA wants, so P never moves between lanes.  V is the PV MFMA's A operand
// (row = dim, k = key): tile t takes the dims 8 * row + t, so lane l's four
// 16-byte loads of rows 4g + i (dims 8r .. 8r+7) hold its A values for all
// eight tiles.  Output: the C layout of tile t leaves lane l dims
// 8 (4g + i) + t of query r, eight consecutive floats per i.  The wavefronts'
// (max, sum, output) triples are merged through LDS in wavefront order:
// M = max m_w, out = sum_w e^(m_w - M) o_w / sum_w e^(m_w - M) l_w.  Under a
// causal mask the tiles of late rows walk many more blocks than early ones;
// split over four wavefronts the longest chain is a quarter as long and four
// times as many wavefronts share the chip.
typedef _Float16 af_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 af_h4 __attribute__((ext_vector_type(4)));
typedef float af_f4 __attribute__((ext_vector_type(4)));
constexpr int AF_WAVES = 4;  // wavefronts per query tile (key-range split)

__device__ __forceinline__ void split_f16(float v, _Float16& hi, _Float16& lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

__global__ __launch_bounds__(64 * AF_WAVES) void attention_prefill_kernel(const float* __restrict__ q, int ldq,
                                                                          const uint16_t* __restrict__ kc,
                                                                          const uint16_t* __restrict__ vc, int pos0,
                                                                          int M, int max_ctx, float scale,
                                                                          float* __restrict__ out, int ldo) {
    __shared__ float s_o[AF_WAVES - 1][32][64];  // (wavefronts 1..: wavefront 0 keeps its own)
    __shared__ float s_m[AF_WAVES][16], s_l[AF_WAVES][16];
    const int h = blockIdx.x, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int m0 = 16 * (int)blockIdx.y;  // (< M: the grid has ceil(M / 16) tiles)
    const int r = lane & 15, g = lane >> 4;
    const int m = m0 + r;
    const int mq = m < M ? m : M - 1;
    const int qpos = pos0 + mq;                          // this lane's query position
    const int jmax = pos0 + (m0 + 15 < M ? m0 + 15 : M - 1);  // the tile's last cache row
    const uint16_t* kh = kc + (size_t)h * max_ctx * HD;
    const uint16_t* vh = vc + (size_t)h * max_ctx * HD;

    // Q^T as the S^T MFMA's B operand: dims 32t + 8g + e of query r
    af_h8 qhi[4], qlo[4];
    const float* qr = q + (size_t)mq * ldq + (size_t)h * HD;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const float4 x0 = *reinterpret_cast<const float4*>(qr + 32 * t + 8 * g);
        const float4 x1 = *reinterpret_cast<const float4*>(qr + 32 * t + 8 * g + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            _Float16 a, b;
            split_f16(xv[e], a, b);
            qhi[t][e] = a;
            qlo[t][e] = b;
        }
    }
    // one block's loads: K row j0 + r (dims 32t + 8g ..), V rows j0 + 4g + i
    // (dims 8r ..); rows past the tile's last are clamped to it (their
    // weights are 0; the row is written, so 0 * v stays 0)
    auto load_blk = [&](int j0, uint4 (&kf)[4], uint4 (&vf)[4]) {
        const int kr = j0 + r < jmax ? j0 + r : jmax;
#pragma unroll
        for (int t = 0; t < 4; t++) kf[t] = *reinterpret_cast<const uint4*>(kh + (size_t)kr * HD + 32 * t + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int vr = j0 + 4 * g + i < jmax ? j0 + 4 * g + i : jmax;
            vf[i] = *reinterpret_cast<const uint4*>(vh + (size_t)vr * HD + 8 * r);
        }
    };
    af_f4 o[8];
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] = af_f4{0.f, 0.f, 0.f, 0.f};
    // (a finite floor: a range whose blocks are all past a row's position
    // keeps m = -1e30, l = 0, o = 0 and weighs 0 in the merge; block 0, live
    // for every row, is in wavefront 0's range)
    float mrun = -1e30f, lrun = 0.0f;
    auto block = [&](int j0, const uint4 (&kf)[4], const uint4 (&vf)[4]) {
        af_f4 st = af_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const af_h8 a = __builtin_bit_cast(af_h8, kf[t]);
            st = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qhi[t], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qlo[t], st, 0, 0, 0);
        }
        float sv[4], bmax = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            sv[i] = j0 + 4 * g + i <= qpos ? st[i] * scale : -__builtin_inff();
            bmax = fmaxf(bmax, sv[i]);
        }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float mnew = fmaxf(mrun, bmax);  // finite (>= the floor)
        const float c = expf(mrun - mnew);     // (0 on the first live block, where lrun = o = 0)
        float p[4], psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p[i] = expf(sv[i] - mnew);
            psum += p[i];
        }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        lrun = lrun * c + psum;
        mrun = mnew;
        af_h4 phi, plo;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            _Float16 a, b;
            split_f16(p[i], a, b);
            phi[i] = a;
            plo[i] = b;
        }
        const uint32_t vw[4][4] = {{vf[0].x, vf[0].y, vf[0].z, vf[0].w}, {vf[1].x, vf[1].y, vf[1].z, vf[1].w},
                                   {vf[2].x, vf[2].y, vf[2].z, vf[2].w}, {vf[3].x, vf[3].y, vf[3].z, vf[3].w}};
#pragma unroll
        for (int t = 0; t < 8; t++) {
            // A (dim row r of tile t, keys 4g + i): half t of each V row's load
            const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;  // high or low halves of two words
            const uint32_t w01 = __builtin_amdgcn_perm(vw[1][t >> 1], vw[0][t >> 1], sel);
            const uint32_t w23 = __builtin_amdgcn_perm(vw[3][t >> 1], vw[2][t >> 1], sel);
            const af_h4 a = __builtin_bit_cast(af_h4, (unsigned long long)w01 | ((unsigned long long)w23 << 32));
            af_f4 ot = o[t] * c;
            ot = __builtin_amdgcn_mfma_f32_16x16x16f16(a, phi, ot, 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, plo, ot, 0, 0, 0);
        }
    };
    // two-block register ring: the next block's loads are in flight while a
    // block is computed (past the last block the ring re-reads its last one)
    // this wavefront's blocks [b0, b1) of the tile's nblk
    const int nblk = jmax / 16 + 1, per = (nblk + AF_WAVES - 1) / AF_WAVES;
    const int b0 = w * per, b1 = min(nblk, b0 + per);
    if (b0 < b1) {  // (wave-uniform)
        const int jlast = 16 * (b1 - 1);
        uint4 ka[4], va[4], kb[4], vb[4];
        int j0 = 16 * b0;
        load_blk(j0, ka, va);
        while (true) {
            load_blk(j0 + 16 <= jlast ? j0 + 16 : j0, kb, vb);
            block(j0, ka, va);
            j0 += 16;
            if (j0 > jlast) break;
            load_blk(j0 + 16 <= jlast ? j0 + 16 : j0, ka, va);
            block(j0, kb, vb);
            j0 += 16;
            if (j0 > jlast) break;
        }
    }
    if (w > 0) {
#pragma unroll
        for (int t = 0; t < 8; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) s_o[w - 1][4 * t + i][lane] = o[t][i];
    }
    if (g == 0) {
        s_m[w][r] = mrun;
        s_l[w][r] = lrun;
    }
    __syncthreads();
    if (w == 0 && m < M) {
        float mx = s_m[0][r];
#pragma unroll
        for (int v = 1; v < AF_WAVES; v++) mx = fmaxf(mx, s_m[v][r]);
        float wt[AF_WAVES], l = 0.0f;
#pragma unroll
        for (int v = 0; v < AF_WAVES; v++) {
            wt[v] = expf(s_m[v][r] - mx);
            l += s_l[v][r] * wt[v];
        }
        const float inv = 1.0f / l;
        float res[32];
#pragma unroll
        for (int k = 0; k < 32; k++) {
            float a = o[k >> 2][k & 3] * wt[0];
#pragma unroll
            for (int v = 1; v < AF_WAVES; v++) a = fmaf(s_o[v - 1][k][lane], wt[v], a);
            res[k] = a * inv;
        }
        float* orow = out + (size_t)m * ldo + (size_t)h * HD;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4* dst = reinterpret_cast<float4*>(orow + 8 * (4 * g + i));
            dst[0] = make_float4(res[i], res[4 + i], res[8 + i], res[12 + i]);
            dst[1] = make_float4(res[16 + i], res[20 + i], res[24 + i], res[28 + i]);
        }
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
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(attention_prefill_kernel, dim3(n_heads, (M + 15) / 16),
                       dim3(64 * AF_WAVES), 0, s, q, ldq, kc, vc, pos0, M, max_ctx, scale, out, ldo);
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
