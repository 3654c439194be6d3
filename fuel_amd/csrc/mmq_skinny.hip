// Quantized matmul for a few activation rows (2 <= M, up to 32 per row group):
// fuel's matmul<T> (k_quants.rs:2284-2331) for T = BlockQ4K / BlockQ6K /
// BlockQ8_0 on int8 MFMA, with each weight block read once from HBM straight
// into registers.
//
// The activation rows are quantized once beforehand (quantize_q8k /
// quantize_q8_0 into the device workspace, SoA: qs [M][K], d [M][K/blk],
// bsums).  A workgroup owns 16 output columns and every row group of up to
// 16*RT rows; its 16 wavefronts split K: wavefront w takes the 256-element
// units w, w+16, ... (one Q4_K / Q6_K superblock, or eight Q8_0 blocks).
// Lane l of a wavefront handles column l%16 and lane group c = l/16: it issues
// exactly the loads of the one-row mat-vec's lane c for that column's block
// (formats.hpp: Q4K/Q6K/Q80::load), so the 64 lanes read the 16 blocks once,
// 16 bytes per load, and build the MFMA B fragments in registers.  The K
// slots of an MFMA step are ordered to match those loads (a dot product does
// not depend on the order of K, as long as A and B agree): lane group c of
// step t holds elements
//   Q4_K  64c + 16t + [0,16)            (nibbles of its two 16-byte qs pieces)
//   Q6_K  128(c>>1) + 32t + 16(c&1) + [0,16)   (its ql / qh pieces, code t)
//   Q8_0  32j + 8c + [0,8) of block j   (v_mfma_i32_16x16x32_i8, one block per MFMA)
// and the A fragments are 16-byte (8-byte) loads of those elements of the
// quantized rows, from L2.  Integer sums per superblock / block are exact:
//   Q4_K  isum = 8*(X.Ba) + X.Bb, msum = X.Bm  (sc = 8a + b; mins broadcast),
//   Q6_K  isum = 128*(X.Wh) + X.Wl            (w = (q-32)*sc = 128 wh + wl),
//   Q8_0  isum = X.Q,
// then one f32 step per superblock (block): y += d_x * (d*isum - dmin*msum).
// At the end the 16 wavefronts' partial tiles are summed through LDS in
// wavefront order (deterministic) and stored.
#include "common.hpp"
#include "formats.hpp"
#include "kernels.hpp"
#include "mfma.hpp"
#include "regb.hpp"

namespace frq {

namespace {

constexpr int SK_COLS = 16;    // output columns per workgroup

// A fragments of unit u for the lane's row tiles: row m0 + 16rt + l%16
// (clamped into [0, M)), bytes aoff(c, t) of the unit.
template <class F, int RT>
__device__ __forceinline__ void sk_load_a(const int8_t* __restrict__ qs, int K, int u, int c, const int (&arow)[RT],
                                          v4i (&a)[RT][F::NA]) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int8_t* p = qs + (size_t)arow[rt] * K + (size_t)u * SK_UNIT;
#pragma unroll
        for (int t = 0; t < F::NA; t++) {
            if constexpr (F::ACT == GGML_Q8_0) {  // blocks 2t, 2t+1: bytes 64t + 8c and 64t + 32 + 8c
                const uint2 lo = *reinterpret_cast<const uint2*>(p + F::aoff(c, t));
                const uint2 hi = *reinterpret_cast<const uint2*>(p + F::aoff(c, t) + 32);
                a[rt][t] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            } else {
                a[rt][t] = *reinterpret_cast<const v4i*>(p + F::aoff(c, t));
            }
        }
    }
}

// A workgroup is one 16-column tile; its NWV wavefronts split K (NWV is
// sized by the launcher so that tiles x NWV wavefronts fill the GPU: 16 for
// N = 4096, fewer for wider matrices, whose wavefronts then stream several
// units each through the register ring).
template <class F, int RT, int NWV>
__global__ __launch_bounds__(64 * NWV) void mmq_skinny_kernel(const uint8_t* __restrict__ W, ActView act,
                                                                    float* __restrict__ y, int M, int N, int K,
                                                                    int ldy, int out_mode) {
    __shared__ float red[NWV][RT][4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane >> 4, l16 = lane & 15;
    const int n0 = blockIdx.x * SK_COLS, m0 = blockIdx.y * 16 * RT;
    const int KU = K / SK_UNIT;
    const int n = n0 + l16 < N ? n0 + l16 : N - 1;  // tail columns re-read a valid row; their outputs are dropped
    const size_t row_bytes = F::ACT == GGML_Q8_0 ? (size_t)(K / QK8_0) * Q8_0_BYTES : (size_t)(K / QK_K) * F::BYTES;
    const uint8_t* wrow = W + (size_t)n * row_bytes;
    int arow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int m = m0 + 16 * rt + l16;
        arow[rt] = m < M ? m : M - 1;
    }
    float facc[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) facc[rt][i] = 0.0f;

    // the lane's output rows (C layout: rows 4c + i of each 16-row tile)
    int orow[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + 16 * rt + 4 * c + i;
            orow[rt][i] = m < M ? m : M - 1;
        }

    // Two-unit register ring: the next unit's weight and activation loads are
    // in flight while the current one is multiplied.  The loads are
    // unconditional (past the last unit a wavefront re-reads its current one,
    // cache-resident), so no branch sits between a load and its use.
    auto step = [&](const typename F::Raw& rw, const v4i(&av)[RT][F::NA], int uu) __attribute__((always_inline)) {
        if constexpr (F::ACT == GGML_Q8_0) {
            const float* dx[RT][4];  // d of blocks 8uu.. of the lane's output rows
            const int KB = K / QK8_0;
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) dx[rt][i] = act.d + (size_t)orow[rt][i] * KB + 8 * uu;
            F::template unit<RT>(rw, [&](int rt, int t) { return av[rt][t]; }, c, dx, facc);
        } else {
            float dx[RT][4];
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) dx[rt][i] = act.d[(size_t)orow[rt][i] * KU + uu];
            F::template unit<RT>(rw, [&](int rt, int t) { return av[rt][t]; }, c, dx, facc);
        }
    };
    typename F::Raw ra, rb;
    v4i aa[RT][F::NA], ab[RT][F::NA];
    int u = wave;
    if (u < KU) {  // (uniform: a wavefront past the last unit only joins the reduction)
        F::load(wrow, u, c, ra);
        sk_load_a<F, RT>(act.qs, K, u, c, arow, aa);
        while (true) {
            int nu = u + NWV < KU ? u + NWV : u;
            F::load(wrow, nu, c, rb);
            sk_load_a<F, RT>(act.qs, K, nu, c, arow, ab);
            step(ra, aa, u);
            if (u + NWV >= KU) break;
            u += NWV;
            nu = u + NWV < KU ? u + NWV : u;
            F::load(wrow, nu, c, ra);
            sk_load_a<F, RT>(act.qs, K, nu, c, arow, aa);
            step(rb, ab, u);
            if (u + NWV >= KU) break;
            u += NWV;
        }
    }

#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[wave][rt][i][lane] = facc[rt][i];
    __syncthreads();
    for (int e = threadIdx.x; e < RT * 4 * 64; e += 64 * NWV) {
        const int rt = e >> 8, i = (e >> 6) & 3, l = e & 63;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; w++) s += red[w][rt][i][l];
        const int m = m0 + 16 * rt + 4 * (l >> 4) + i, nn = n0 + (l & 15);
        if (m < M && nn < N) store_out(y, (size_t)m * ldy + nn, s, out_mode);
    }
}

template <class F, int RT, int NWV>
hipError_t launch_sk(const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy, hipStream_t s,
                     int yh) {
    const dim3 grid((N + SK_COLS - 1) / SK_COLS, (M + 16 * RT - 1) / (16 * RT));
    hipLaunchKernelGGL((mmq_skinny_kernel<F, RT, NWV>), grid, dim3(64 * NWV), 0, s, w, act, y, M, N, K, ldy,
                       yh);
    return hipGetLastError();
}

// K split: about 16 wavefronts per CU over the whole grid (the tiles of every
// row group), at most 16 per tile and no more than the tile has units.
int sk_split(int tiles, int KU, int num_cus) {
    const long target = 16L * num_cus;
    int nwv = 16;
    while (nwv > 2 && ((long)tiles * nwv / 2 >= target || nwv / 2 >= KU)) nwv /= 2;
    return nwv;
}

template <class F, int RT>
hipError_t launch_sk_rt(const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy, int num_cus,
                        hipStream_t s, int yh) {
    const int tiles = (N + SK_COLS - 1) / SK_COLS * ((M + 16 * RT - 1) / (16 * RT));
    // (two row tiles: at most 8 wavefronts, 512 threads, for their registers)
    const int nwv = sk_split(tiles, K / SK_UNIT, num_cus);
    switch (RT == 2 && nwv > 8 ? 8 : nwv) {
        case 16: return launch_sk<F, RT, RT == 2 ? 8 : 16>(w, act, y, M, N, K, ldy, s, yh);
        case 8: return launch_sk<F, RT, 8>(w, act, y, M, N, K, ldy, s, yh);
        case 4: return launch_sk<F, RT, 4>(w, act, y, M, N, K, ldy, s, yh);
        default: return launch_sk<F, RT, 2>(w, act, y, M, N, K, ldy, s, yh);
    }
}

template <class F>
hipError_t launch_sk_fmt(const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy, int num_cus,
                         hipStream_t s, int yh) {
    return M <= 16 ? launch_sk_rt<F, 1>(w, act, y, M, N, K, ldy, num_cus, s, yh)
                   : launch_sk_rt<F, 2>(w, act, y, M, N, K, ldy, num_cus, s, yh);
}

}  // namespace

bool mmq_skinny_supported(int dtype, int K) {
    return (dtype == GGML_Q4K || dtype == GGML_Q6K || dtype == GGML_Q8_0) && K > 0 && K % SK_UNIT == 0;
}

hipError_t launch_mmq_skinny(int dtype, const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy,
                             int num_cus, hipStream_t s, int out_mode) {
    if (!mmq_skinny_supported(dtype, K) || M < 1 || N < 1) return hipErrorInvalidValue;
    switch (dtype) {
        case GGML_Q4K: return launch_sk_fmt<SkQ4K>(w, act, y, M, N, K, ldy, num_cus, s, out_mode);
        case GGML_Q6K: return launch_sk_fmt<SkQ6K>(w, act, y, M, N, K, ldy, num_cus, s, out_mode);
        default: return launch_sk_fmt<SkQ80>(w, act, y, M, N, K, ldy, num_cus, s, out_mode);
    }
}

}  // namespace frq
