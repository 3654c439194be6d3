// Quantized mat-vec for decode-sized M (fuel's matmul<T>, k_quants.rs:2284-2331,
// for T = BlockQ4K / BlockQ6K / BlockQ8_0 against Q8K / Q8_0 activations).
//
// Mapping (wave64): a weight block is handled by LPB consecutive lanes; one
// wavefront covers 64/LPB blocks of the same weight row per step and walks its
// rows with a grid stride.  Each lane keeps its slice of the quantized
// activation row in registers for the whole launch (activation-stationary),
// so HBM traffic is the weight stream plus one activation read per wave.
// Weight bytes arrive as 128-bit loads; scales/mins are unpacked in registers;
// the integer block sums use v_dot4_i32_i8; the row result is a wave64
// reduction.
//
// The integer stage of every block (isum, msum below) is exactly the integer
// sum of vec_dot_unopt (k_quants.rs:1388-1468, 1946-2003, 674-692); the f32
// combination y += d_w*d_x*isum - dmin_w*d_x*msum is the only rounding step.
#include "common.hpp"
#include "kernels.hpp"

namespace frq {

// ------------------------------------------------------------------------
// Q4K: 4 lanes per 144-byte superblock.  Lane c (0..3) owns quant bytes
// qs[32c..32c+32): low nibbles are elements 64c..64c+31 (sub-block 2c), high
// nibbles are 64c+32..64c+63 (sub-block 2c+1)  (k_quants.rs:1603-1620).
// ------------------------------------------------------------------------
struct Q4K {
    static constexpr int LPB = 4;
    static constexpr int BYTES = Q4K_BYTES;
    static constexpr int ELEMS = QK_K;
    struct Act {
        uint4 a[4];   // q8 of elements 64c + 0..63
        int bs_lo;    // bsums[4c] + bsums[4c+1]
        int bs_hi;    // bsums[4c+2] + bsums[4c+3]
        float d;
    };
    __device__ static void load_act(const ActView& act, int m, int K, int b, int c, Act& r) {
        const int KB = K / QK_K;
        const uint4* q = reinterpret_cast<const uint4*>(act.qs + (size_t)m * K + (size_t)b * QK_K + 64 * c);
        r.a[0] = q[0]; r.a[1] = q[1]; r.a[2] = q[2]; r.a[3] = q[3];
        const int16_t* bs = act.bsums + ((size_t)m * KB + b) * 16 + 4 * c;
        r.bs_lo = (int)bs[0] + (int)bs[1];
        r.bs_hi = (int)bs[2] + (int)bs[3];
        r.d = act.d[(size_t)m * KB + b];
    }
    // Integer partials of this lane's 64 elements, plus the block's d / dmin.
    __device__ static void partial(const uint8_t* blk, const Act& x, int c, int& isum, int& msum,
                                   float& dw, float& dmw) {
        const uint4 hd = *reinterpret_cast<const uint4*>(blk);
        const uint4 q0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * c);
        const uint4 q1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * c);
        // 12 packed bytes -> 8 six-bit scales and 8 mins (get_scale_min_k4,
        // utils.rs:50-60), as four words of bytes.
        const uint32_t s0 = hd.y, s1 = hd.z, s2 = hd.w;
        const uint32_t sc_a = s0 & 0x3f3f3f3fu;                                        // scales 0..3
        const uint32_t sc_b = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);   // scales 4..7
        const uint32_t mn_a = s1 & 0x3f3f3f3fu;                                        // mins 0..3
        const uint32_t mn_b = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);  // mins 4..7
        const uint32_t scw = c < 2 ? sc_a : sc_b;
        const uint32_t mnw = c < 2 ? mn_a : mn_b;
        const uint32_t sh = 16u * (uint32_t)(c & 1);
        const int sc_lo = (int)((scw >> sh) & 0xffu), sc_hi = (int)((scw >> (sh + 8)) & 0xffu);
        const int m_lo = (int)((mnw >> sh) & 0xffu), m_hi = (int)((mnw >> (sh + 8)) & 0xffu);
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t alo[8] = {x.a[0].x, x.a[0].y, x.a[0].z, x.a[0].w, x.a[1].x, x.a[1].y, x.a[1].z, x.a[1].w};
        const uint32_t ahi[8] = {x.a[2].x, x.a[2].y, x.a[2].z, x.a[2].w, x.a[3].x, x.a[3].y, x.a[3].z, x.a[3].w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo = dot4(w[i] & 0x0f0f0f0fu, alo[i], lo);
            hi = dot4((w[i] >> 4) & 0x0f0f0f0fu, ahi[i], hi);
        }
        isum = sc_lo * lo + sc_hi * hi;
        msum = m_lo * x.bs_lo + m_hi * x.bs_hi;
        dw = f16_to_f32(hd.x & 0xffffu);
        dmw = f16_to_f32(hd.x >> 16);
    }
};

// ------------------------------------------------------------------------
// Q6K: 4 lanes per 210-byte superblock.  Lane c -> half hh = c>>1 (elements
// 128hh..128hh+127) and column offset l0 = 16*(c&1); it owns the 64 elements
// 128hh + 32*qd + l0 + [0,16) for qd = 0..3, built from ql[64hh+l0..+16]
// (qd 0 low / qd 2 high nibbles), ql[64hh+32+l0..+16] (qd 1 / qd 3) and
// qh[32hh+l0..+16] (2 bits per qd)  (k_quants.rs:2170-2186).  Group scale of
// (qd) is scales[8hh + 2qd + (c&1)].  Blocks are only 2-byte aligned.
// ------------------------------------------------------------------------
struct Q6K {
    static constexpr int LPB = 4;
    static constexpr int BYTES = Q6K_BYTES;
    static constexpr int ELEMS = QK_K;
    struct Act {
        uint4 a[4];  // q8 of the lane's 4 groups of 16
        int bs[4];   // bsums of those groups
        float d;
    };
    __device__ static void load_act(const ActView& act, int m, int K, int b, int c, Act& r) {
        const int KB = K / QK_K;
        const int hh = c >> 1, l0 = 16 * (c & 1);
        const int8_t* q = act.qs + (size_t)m * K + (size_t)b * QK_K + 128 * hh + l0;
        const int16_t* bs = act.bsums + ((size_t)m * KB + b) * 16 + 8 * hh + (c & 1);
#pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            r.a[qd] = *reinterpret_cast<const uint4*>(q + 32 * qd);
            r.bs[qd] = bs[2 * qd];
        }
        r.d = act.d[(size_t)m * KB + b];
    }
    __device__ static void partial(const uint8_t* blk, const Act& x, int c, int& isum, int& msum,
                                   float& dw, float& dmw) {
        const int hh = c >> 1, l0 = 16 * (c & 1);
        const uint4 la = load16_a2(blk + 64 * hh + l0);
        const uint4 lb = load16_a2(blk + 64 * hh + 32 + l0);
        const uint4 qh = load16_a2(blk + 128 + 32 * hh + l0);
        // scales[8hh .. 8hh+8) and d (bytes 192..209)
        const uint2 scw = load8_a2(blk + 192 + 8 * hh);
        const uint32_t dbits = load_u16(blk + 208);
        const uint32_t wa[4] = {la.x, la.y, la.z, la.w};
        const uint32_t wb[4] = {lb.x, lb.y, lb.z, lb.w};
        const uint32_t wh[4] = {qh.x, qh.y, qh.z, qh.w};
        const uint32_t a0[4] = {x.a[0].x, x.a[0].y, x.a[0].z, x.a[0].w};
        const uint32_t a1[4] = {x.a[1].x, x.a[1].y, x.a[1].z, x.a[1].w};
        const uint32_t a2[4] = {x.a[2].x, x.a[2].y, x.a[2].z, x.a[2].w};
        const uint32_t a3[4] = {x.a[3].x, x.a[3].y, x.a[3].z, x.a[3].w};
        // Unsigned 6-bit codes u in [0, 64): sum (u-32)*q8 = dot(u, q8) - 32*bsum.
        int p0 = 0, p1 = 0, p2 = 0, p3 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t u0 = (wa[i] & 0x0f0f0f0fu) | ((wh[i] & 0x03030303u) << 4);
            const uint32_t u1 = (wb[i] & 0x0f0f0f0fu) | (((wh[i] >> 2) & 0x03030303u) << 4);
            const uint32_t u2 = ((wa[i] >> 4) & 0x0f0f0f0fu) | (((wh[i] >> 4) & 0x03030303u) << 4);
            const uint32_t u3 = ((wb[i] >> 4) & 0x0f0f0f0fu) | (((wh[i] >> 6) & 0x03030303u) << 4);
            p0 = dot4(u0, a0[i], p0);
            p1 = dot4(u1, a1[i], p1);
            p2 = dot4(u2, a2[i], p2);
            p3 = dot4(u3, a3[i], p3);
        }
        p0 -= 32 * x.bs[0];
        p1 -= 32 * x.bs[1];
        p2 -= 32 * x.bs[2];
        p3 -= 32 * x.bs[3];
        // scales bytes j = 2qd + (c&1) of the 8-byte window, sign-extended
        const uint32_t sel = (uint32_t)(c & 1) * 8u;
        const int sc0 = (int)(int8_t)((scw.x >> sel) & 0xffu);
        const int sc1 = (int)(int8_t)((scw.x >> (sel + 16)) & 0xffu);
        const int sc2 = (int)(int8_t)((scw.y >> sel) & 0xffu);
        const int sc3 = (int)(int8_t)((scw.y >> (sel + 16)) & 0xffu);
        isum = sc0 * p0 + sc1 * p1 + sc2 * p2 + sc3 * p3;
        msum = 0;
        dw = f16_to_f32(dbits);
        dmw = 0.0f;
    }
};

// ------------------------------------------------------------------------
// Q8_0: 2 lanes per 34-byte block; lane hf owns qs[16hf..16hf+16).
// ------------------------------------------------------------------------
struct Q80 {
    static constexpr int LPB = 2;
    static constexpr int BYTES = Q8_0_BYTES;
    static constexpr int ELEMS = QK8_0;
    struct Act {
        uint4 a;
        float d;
    };
    __device__ static void load_act(const ActView& act, int m, int K, int b, int c, Act& r) {
        const int KB = K / QK8_0;
        r.a = *reinterpret_cast<const uint4*>(act.qs + (size_t)m * K + (size_t)b * QK8_0 + 16 * c);
        r.d = act.d[(size_t)m * KB + b];
    }
    __device__ static void partial(const uint8_t* blk, const Act& x, int c, int& isum, int& msum,
                                   float& dw, float& dmw) {
        const uint4 q = load16_a2(blk + 2 + 16 * c);
        int s = 0;
        s = dot4(q.x, x.a.x, s);
        s = dot4(q.y, x.a.y, s);
        s = dot4(q.z, x.a.z, s);
        s = dot4(q.w, x.a.w, s);
        isum = s;
        msum = 0;
        dw = f16_to_f32(load_u16(blk));
        dmw = 0.0f;
    }
};

// ------------------------------------------------------------------------
// Mat-vec kernel.  SPL = activation slots cached per lane (ceil(KB / BPW));
// SPL == 0 selects the uncached variant that re-reads activations (L1/L2).
// ------------------------------------------------------------------------
template <class F, int SPL>
__global__ __launch_bounds__(256) void mmvq_kernel(const uint8_t* __restrict__ W, ActView act,
                                                   float* __restrict__ y, int N, int K, int ldy) {
    constexpr int BPW = 64 / F::LPB;  // blocks per wavefront step
    const int m = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int gi = lane / F::LPB, c = lane % F::LPB;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * (blockDim.x >> 6);
    const int KB = K / F::ELEMS;
    const size_t row_bytes = (size_t)KB * F::BYTES;

    if constexpr (SPL > 0) {
        typename F::Act xa[SPL];
#pragma unroll
        for (int s = 0; s < SPL; s++) {
            const int b = gi + BPW * s;
            if (b < KB) F::load_act(act, m, K, b, c, xa[s]);
        }
        for (int row = wave; row < N; row += nwaves) {
            const uint8_t* wr = W + (size_t)row * row_bytes;
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < SPL; s++) {
                const int b = gi + BPW * s;
                if (b < KB) {
                    int isum, msum;
                    float dw, dmw;
                    F::partial(wr + (size_t)b * F::BYTES, xa[s], c, isum, msum, dw, dmw);
                    const float dx = xa[s].d;
                    acc = fmaf(dw * dx, (float)isum, acc);
                    acc = fmaf(-(dmw * dx), (float)msum, acc);
                }
            }
            acc = wave_sum(acc);
            if (lane == 0) y[(size_t)m * ldy + row] = acc;
        }
    } else {
        for (int row = wave; row < N; row += nwaves) {
            const uint8_t* wr = W + (size_t)row * row_bytes;
            float acc = 0.0f;
            for (int b = gi; b < KB; b += BPW) {
                typename F::Act xa;
                F::load_act(act, m, K, b, c, xa);
                int isum, msum;
                float dw, dmw;
                F::partial(wr + (size_t)b * F::BYTES, xa, c, isum, msum, dw, dmw);
                acc = fmaf(dw * xa.d, (float)isum, acc);
                acc = fmaf(-(dmw * xa.d), (float)msum, acc);
            }
            acc = wave_sum(acc);
            if (lane == 0) y[(size_t)m * ldy + row] = acc;
        }
    }
}

template <class F>
static hipError_t launch_fmt(const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy,
                             hipStream_t s, int num_cus) {
    constexpr int BPW = 64 / F::LPB;
    const int KB = K / F::ELEMS;
    const int spl = (KB + BPW - 1) / BPW;
    // Enough waves to cover the rows, capped at 16 waves per CU per activation row.
    int waves = N;
    const int cap = num_cus * 16;
    if (waves > cap) waves = cap;
    int blocks = (waves + 3) / 4;
    if (blocks < 1) blocks = 1;
    dim3 grid(blocks, M), block(256);
#define FRQ_CASE(S)                                                                   \
    case S:                                                                           \
        hipLaunchKernelGGL((mmvq_kernel<F, S>), grid, block, 0, s, w, act, y, N, K, ldy); \
        break;
    switch (spl) {
        FRQ_CASE(1)
        FRQ_CASE(2)
        FRQ_CASE(3)
        FRQ_CASE(4)
        FRQ_CASE(5)
        FRQ_CASE(6)
        FRQ_CASE(7)
        FRQ_CASE(8)
        default:
            hipLaunchKernelGGL((mmvq_kernel<F, 0>), grid, block, 0, s, w, act, y, N, K, ldy);
            break;
    }
#undef FRQ_CASE
    return hipGetLastError();
}

hipError_t launch_mmvq(int dtype, const uint8_t* w, ActView act, float* y, int M, int N, int K,
                       int ldy, hipStream_t s, int num_cus) {
    switch (dtype) {
        case GGML_Q4K: return launch_fmt<Q4K>(w, act, y, M, N, K, ldy, s, num_cus);
        case GGML_Q6K: return launch_fmt<Q6K>(w, act, y, M, N, K, ldy, s, num_cus);
        case GGML_Q8_0: return launch_fmt<Q80>(w, act, y, M, N, K, ldy, s, num_cus);
        default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------------------
// Integer tap: isum/msum of every (m, n, block), from the same per-lane
// partials the mat-vec uses, summed over the LPB lanes of the block.
// grid = (ceil(N*KB / (64/LPB)), M), 64 threads.
// ------------------------------------------------------------------------
template <class F>
__global__ __launch_bounds__(64) void block_isums_kernel(const uint8_t* __restrict__ W, ActView act,
                                                         int32_t* __restrict__ isum,
                                                         int32_t* __restrict__ msum, int N, int K) {
    constexpr int BPW = 64 / F::LPB;
    const int m = blockIdx.y, lane = threadIdx.x;
    const int KB = K / F::ELEMS;
    const long long flat = (long long)blockIdx.x * BPW + lane / F::LPB;  // n * KB + b
    const int c = lane % F::LPB;
    const bool live = flat < (long long)N * KB;
    int is = 0, ms = 0;
    if (live) {
        const int n = (int)(flat / KB), b = (int)(flat % KB);
        typename F::Act xa;
        F::load_act(act, m, K, b, c, xa);
        float dw, dmw;
        F::partial(W + ((size_t)n * KB + b) * F::BYTES, xa, c, is, ms, dw, dmw);
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

hipError_t launch_block_isums(int dtype, const uint8_t* w, ActView act, int32_t* isum,
                              int32_t* msum, int M, int N, int K, hipStream_t s) {
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
