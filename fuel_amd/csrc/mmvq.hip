// Quantized mat-vec for decode-sized M: fuel's matmul<T> (k_quants.rs:2284-2331)
// for T = BlockQ4K / BlockQ6K / BlockQ8_0, including the activation quantize
// step, in one kernel.
//
// Each workgroup first quantizes its activation row (f32 -> Q8K / Q8_0, the
// bit-exact routine of q8.hpp) into LDS, while the first weight row's loads
// are already in flight.  Then every wavefront walks weight rows with a grid
// stride: LPB lanes per block, 64/LPB blocks of one row per step, the lane's
// activation slices held in registers for the whole launch (activation-
// stationary), the next row's 128-bit weight loads issued before the current
// row is reduced.  Scales/mins are unpacked in registers, the integer block
// sums use v_dot4_i32_i8 and each row ends in a wave64 reduction.
//
// The only rounding after the exact integer stage is the f32 combination
// y += d_w*d_x*isum - dmin_w*d_x*msum.
#include "common.hpp"
#include "formats.hpp"
#include "kernels.hpp"
#include "q8.hpp"

namespace frq {

template <class F, int SPL, int WG>
__global__ __launch_bounds__(WG) void qmv_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                 float* __restrict__ y, int N, int K, int ldy) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NW = WG / 64;
    constexpr int BPW = 64 / F::LPB;  // blocks of one row per wavefront step
    const int m = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gi = lane / F::LPB, c = lane % F::LPB;
    const int KB = K / F::ELEMS;
    const int KBa = F::ACT == GGML_Q8K ? K / QK_K : K / QK8_0;
    const size_t row_bytes = (size_t)KB * F::BYTES;
    int8_t* s_qs = reinterpret_cast<int8_t*>(smem);
    float* s_d = reinterpret_cast<float*>(smem + K);
    int16_t* s_bs = reinterpret_cast<int16_t*>(smem + K + 4 * KBa);
    const int nw = gridDim.x * NW;
    int row = blockIdx.x * NW + w;

    typename F::Raw cur[SPL > 0 ? SPL : 1];
    if constexpr (SPL > 0) {
        if (row < N) {
#pragma unroll
            for (int s = 0; s < SPL; s++) {
                const int b = gi + BPW * s;
                if (b < KB) F::load(W + (size_t)row * row_bytes + (size_t)b * F::BYTES, c, cur[s]);
            }
        }
    }

    const float* xr = x + (size_t)m * K;
    if constexpr (F::ACT == GGML_Q8K) q8k_quantize_row(xr, K, s_qs, s_d, s_bs, w, NW, lane);
    else q8_0_quantize_row(xr, K, s_qs, s_d, w, NW, lane);
    __syncthreads();

    if constexpr (SPL > 0) {
        typename F::Act xa[SPL];
#pragma unroll
        for (int s = 0; s < SPL; s++) {
            const int b = gi + BPW * s;
            if (b < KB) F::load_act(s_qs, s_d, s_bs, b, c, xa[s]);
        }
        while (row < N) {
            const int nrow = row + nw;
            typename F::Raw nxt[SPL];
            if (nrow < N) {
#pragma unroll
                for (int s = 0; s < SPL; s++) {
                    const int b = gi + BPW * s;
                    if (b < KB) F::load(W + (size_t)nrow * row_bytes + (size_t)b * F::BYTES, c, nxt[s]);
                }
            }
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < SPL; s++) {
                const int b = gi + BPW * s;
                if (b < KB) {
                    int isum, msum;
                    float dw, dmw;
                    F::dot(cur[s], xa[s], c, isum, msum, dw, dmw);
                    acc = fmaf(dw * xa[s].d, (float)isum, acc);
                    acc = fmaf(-(dmw * xa[s].d), (float)msum, acc);
                }
            }
            acc = wave_sum(acc);
            if (lane == 0) y[(size_t)m * ldy + row] = acc;
#pragma unroll
            for (int s = 0; s < SPL; s++) cur[s] = nxt[s];
            row = nrow;
        }
    } else {
        for (; row < N; row += nw) {
            const uint8_t* wr = W + (size_t)row * row_bytes;
            float acc = 0.0f;
            for (int b = gi; b < KB; b += BPW) {
                typename F::Act xa;
                typename F::Raw r;
                F::load_act(s_qs, s_d, s_bs, b, c, xa);
                F::load(wr + (size_t)b * F::BYTES, c, r);
                int isum, msum;
                float dw, dmw;
                F::dot(r, xa, c, isum, msum, dw, dmw);
                acc = fmaf(dw * xa.d, (float)isum, acc);
                acc = fmaf(-(dmw * xa.d), (float)msum, acc);
            }
            acc = wave_sum(acc);
            if (lane == 0) y[(size_t)m * ldy + row] = acc;
        }
    }
}

namespace {

template <class F, int SPL, int WG>
hipError_t launch_qmv(const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy, hipStream_t s,
                      int num_cus) {
    constexpr int NW = WG / 64;
    static int occ = -1;  // resident workgroups per CU for this instantiation
    if (occ < 0) {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, qmv_kernel<F, SPL, WG>, WG, 16384) != hipSuccess || o < 1)
            o = 1;
        occ = o;
    }
    const int kba = F::ACT == GGML_Q8K ? K / QK_K : K / QK8_0;
    const size_t lds = (size_t)K + 4u * kba + (F::ACT == GGML_Q8K ? 32u * kba : 0u);
    if (lds > 65536) return hipErrorInvalidValue;
    const int need = (N + NW - 1) / NW;
    int cap = num_cus * occ / (M > 0 ? M : 1);
    if (cap < 1) cap = 1;
    const int gx = need < cap ? need : cap;
    hipLaunchKernelGGL((qmv_kernel<F, SPL, WG>), dim3(gx, M), dim3(WG), lds, s, w, x, y, N, K, ldy);
    return hipGetLastError();
}

template <class F>
hipError_t launch_fmt(const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy, hipStream_t s,
                      int num_cus) {
    constexpr int BPW = 64 / F::LPB;
    const int KB = K / F::ELEMS;
    const int spl = (KB + BPW - 1) / BPW;
    // Workgroup size by register footprint: the widest that needs no spills.
    constexpr bool wide = sizeof(typename F::Raw) > 64;  // Q6K carries realignment dwords
    switch (spl) {
        case 1: return launch_qmv<F, 1, 1024>(w, x, y, M, N, K, ldy, s, num_cus);
        case 2: return launch_qmv<F, 2, wide ? 512 : 1024>(w, x, y, M, N, K, ldy, s, num_cus);
        case 3: return launch_qmv<F, 3, 512>(w, x, y, M, N, K, ldy, s, num_cus);
        case 4: return launch_qmv<F, 4, wide ? 256 : 512>(w, x, y, M, N, K, ldy, s, num_cus);
        case 5: return launch_qmv<F, 5, 256>(w, x, y, M, N, K, ldy, s, num_cus);
        case 6: return launch_qmv<F, 6, 256>(w, x, y, M, N, K, ldy, s, num_cus);
        default: return launch_qmv<F, 0, 256>(w, x, y, M, N, K, ldy, s, num_cus);
    }
}

}  // namespace

hipError_t launch_qmv(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                      hipStream_t s, int num_cus) {
    switch (dtype) {
        case GGML_Q4K: return launch_fmt<Q4K>(w, x, y, M, N, K, ldy, s, num_cus);
        case GGML_Q6K: return launch_fmt<Q6K>(w, x, y, M, N, K, ldy, s, num_cus);
        case GGML_Q8_0: return launch_fmt<Q80>(w, x, y, M, N, K, ldy, s, num_cus);
        default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------------------
// Integer tap: isum/msum of every (m, n, block) from the same per-lane
// partials as the mat-vec, summed over the LPB lanes of each block.
// grid = (ceil(N*KB / (64/LPB)), M), 64 threads; activations from an ActView.
// ------------------------------------------------------------------------
template <class F>
__global__ __launch_bounds__(64) void block_isums_kernel(const uint8_t* __restrict__ W, ActView act,
                                                         int32_t* __restrict__ isum, int32_t* __restrict__ msum,
                                                         int N, int K) {
    constexpr int BPW = 64 / F::LPB;
    const int m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / F::ELEMS;
    const int KBa = F::ACT == GGML_Q8K ? K / QK_K : K / QK8_0;
    const long long flat = (long long)blockIdx.x * BPW + lane / F::LPB;  // n * KB + b
    const int c = lane % F::LPB;
    const bool live = flat < (long long)N * KB;
    int is = 0, ms = 0;
    if (live) {
        const int n = (int)(flat / KB), b = (int)(flat % KB);
        typename F::Act xa;
        F::load_act(act.qs + (size_t)m * K, act.d + (size_t)m * KBa,
                    act.bsums ? act.bsums + (size_t)m * KBa * 16 : nullptr, b, c, xa);
        typename F::Raw r;
        F::load(W + ((size_t)n * KB + b) * F::BYTES, c, r);
        float dw, dmw;
        F::dot(r, xa, c, is, ms, dw, dmw);
    }
#pragma unroll
    for (int off = 1; off < F::LPB; off <<= 1) {
        is += __shfl_xor(is, off, 64);
        ms += __shfl_xor(ms, off, 64);
    }
    if (live && c == 0) {
        const size_t o = (size_t)m * N * KB + (size_t)flat;
        isum[o] = is;
        msum[o] = ms;
    }
}

hipError_t launch_block_isums(int dtype, const uint8_t* w, ActView act, int32_t* isum, int32_t* msum, int M,
                              int N, int K, hipStream_t s) {
    auto go = [&](auto fmt) {
        using F = decltype(fmt);
        constexpr int BPW = 64 / F::LPB;
        const long long total = (long long)N * (K / F::ELEMS);
        dim3 grid((unsigned)((total + BPW - 1) / BPW), M);
        hipLaunchKernelGGL(block_isums_kernel<F>, grid, dim3(64), 0, s, w, act, isum, msum, N, K);
        return hipGetLastError();
    };
    switch (dtype) {
        case GGML_Q4K: return go(Q4K{});
        case GGML_Q6K: return go(Q6K{});
        case GGML_Q8_0: return go(Q80{});
        default: return hipErrorInvalidValue;
    }
}

}  // namespace frq
