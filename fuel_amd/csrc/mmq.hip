// Batched / prefill quantized matmul (M >= 16) on gfx950 int8 MFMA:
// fuel's matmul<BlockQ4K> (k_quants.rs:2284-2331) for many activation rows.
//
// Exact integer formulation.  Per superblock b, with q4 the weight nibbles,
// sc_j / m_j the 6-bit scale / min of sub-block j and q8 the Q8K activation:
//   isum = sum_j sc_j * sum_{e in j} q4_e q8_e ,  msum = sum_j m_j * sum_{e in j} q8_e
// A 6-bit scale times a nibble does not fit int8, so sc_j = 8*a_j + b_j with
// a_j, b_j <= 7: q4*a_j and q4*b_j are <= 105 and a dword holding four nibbles
// can be multiplied by a_j without carries between its bytes.  Then
//   isum = 8 * (X . Ba) + (X . Bb),   msum = X . Bm
// with Ba = q4*a_j, Bb = q4*b_j, Bm = m_j (broadcast over the sub-block): three
// int8 GEMMs over K = 256 per superblock on v_mfma_i32_16x16x64_i8, exact in
// int32, followed by one f32 step y += d_w*d_x*isum - dmin_w*d_x*msum.
//
// Workgroup: 4 wavefronts on a WM x WN grid, each owning RT x CT tiles of 16x16
// outputs.  Per superblock the workgroup stages the quantized activation rows
// (272-byte LDS row stride) and the raw weight blocks of its columns in LDS;
// each lane then builds its B fragments in registers from the raw nibbles.
#include "common.hpp"
#include "kernels.hpp"

namespace frq {

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int A_STRIDE = QK_K + 16;  // LDS bytes per activation row per superblock

template <int RT, int CT, int WM, int WN>
struct MmqTile {
    static constexpr int NT = 64 * WM * WN;
    static constexpr int BM = 16 * RT * WM, BN = 16 * CT * WN;
    static constexpr int A_CH = BM * 16;                   // 16-byte activation chunks per superblock
    static constexpr int W_CH = BN * 9;                    // 16-byte weight chunks per superblock
    static constexpr int A_PT = (A_CH + NT - 1) / NT;      // per thread
    static constexpr int W_PT = (W_CH + NT - 1) / NT;
};

// Global -> register prefetch of one superblock's activation rows and raw
// weight blocks.  arow: this thread's activation row per chunk (-1: padding
// row, staged as zeros); wrow: its weight row base per chunk; dxrow: the row
// whose scale it stages (-1: none).
template <int RT, int CT, int WM, int WN>
__device__ __forceinline__ void mmq_fetch(const ActView& act, int K, int b, int tid,
                                          const int (&arow)[MmqTile<RT, CT, WM, WN>::A_PT],
                                          const uint8_t* const (&wrow)[MmqTile<RT, CT, WM, WN>::W_PT], int dxrow,
                                          uint4 (&ra)[MmqTile<RT, CT, WM, WN>::A_PT],
                                          uint4 (&rw)[MmqTile<RT, CT, WM, WN>::W_PT], float& rdx) {
    using T = MmqTile<RT, CT, WM, WN>;
    const int KB = K / QK_K;
#pragma unroll
    for (int i = 0; i < T::A_PT; i++) {
        const int ch = (tid + i * T::NT) & 15;
        ra[i] = uint4{0u, 0u, 0u, 0u};
        if (arow[i] >= 0)
            ra[i] = *reinterpret_cast<const uint4*>(act.qs + (size_t)arow[i] * K + (size_t)b * QK_K + 16 * ch);
    }
#pragma unroll
    for (int i = 0; i < T::W_PT; i++) {
        const int idx = tid + i * T::NT;
        rw[i] = uint4{0u, 0u, 0u, 0u};  // (a conditionally-set array would live in scratch)
        if (idx < T::W_CH) rw[i] = *reinterpret_cast<const uint4*>(wrow[i] + (size_t)b * Q4K_BYTES + 16 * (idx % 9));
    }
    rdx = dxrow >= 0 ? act.d[(size_t)dxrow * KB + b] : 0.0f;
}

template <int RT, int CT, int WM, int WN>
__device__ __forceinline__ void mmq_stage(int8_t* s_a, uint8_t* s_w, float* s_dx, int tid,
                                          const uint4 (&ra)[MmqTile<RT, CT, WM, WN>::A_PT],
                                          const uint4 (&rw)[MmqTile<RT, CT, WM, WN>::W_PT], float rdx) {
    using T = MmqTile<RT, CT, WM, WN>;
#pragma unroll
    for (int i = 0; i < T::A_PT; i++) {
        const int idx = tid + i * T::NT;
        if (idx < T::A_CH) *reinterpret_cast<uint4*>(s_a + (idx >> 4) * A_STRIDE + 16 * (idx & 15)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < T::W_PT; i++) {
        const int idx = tid + i * T::NT;
        if (idx < T::W_CH) *reinterpret_cast<uint4*>(s_w + (idx / 9) * Q4K_BYTES + 16 * (idx % 9)) = rw[i];
    }
    if (tid < T::BM) s_dx[tid] = rdx;
}

// grid = (M tiles, N tiles, K splits).  With ksplit > 1 each workgroup sums a
// contiguous range of superblocks into part[split][M][N]; mmq_reduce_kernel
// adds the splits in order afterwards (deterministic).
// GROUPED (MoE): workgroup x is tile x of the expert-sorted rows (g.tile_*);
// its rows end at its expert's end offset, its weights are that expert's, and
// activation row m is g.x_row[m] (gathered token rows) when x_row is set.
template <int RT, int CT, int WM, int WN, bool GROUPED>
__global__ __launch_bounds__(64 * WM * WN) void mmq_q4k_kernel(const uint8_t* __restrict__ W, ActView act,
                                                               float* __restrict__ y, int M, int N, int K,
                                                               int ldy, MmqGroup g) {
    using T = MmqTile<RT, CT, WM, WN>;
    constexpr int BM = T::BM, BN = T::BN;
    __shared__ __align__(16) int8_t s_a[BM * A_STRIDE];
    __shared__ __align__(16) uint8_t s_w[BN * Q4K_BYTES];
    __shared__ float s_dx[BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int n0 = blockIdx.y * BN;
    const int KB = K / QK_K;
    const size_t row_bytes = (size_t)KB * Q4K_BYTES;
    const int nsplit = gridDim.z;
    const int b0 = (int)((long long)KB * blockIdx.z / nsplit), b1 = (int)((long long)KB * (blockIdx.z + 1) / nsplit);
    const int l16 = lane & 15, kb = lane >> 4;

    int m0 = blockIdx.x * BM, mend = M, n_split = N;
    const uint8_t* W1 = W;
    const uint8_t* W2 = W;
    const int* x_row = nullptr;
    if constexpr (GROUPED) {
        const int tile = blockIdx.x;
        if (tile >= *g.ntiles) return;  // uniform: the tile table is shorter than the grid bound
        const int e = g.tile_expert[tile];
        m0 = g.tile_row0[tile];
        mend = g.expert_offsets[e + 1];
        W1 = W + (size_t)e * g.expert_bytes;
        W2 = g.w2 ? g.w2 + (size_t)e * g.expert_bytes : W1;
        if (g.w2) n_split = g.n_split;
        x_row = g.x_row;
    }
    int arow[T::A_PT];
#pragma unroll
    for (int i = 0; i < T::A_PT; i++) {
        const int idx = tid + i * T::NT;
        const int m = m0 + (idx >> 4);
        arow[i] = idx < T::A_CH && m < mend ? (x_row ? x_row[m] : m) : -1;
    }
    const int dxrow = tid < BM && m0 + tid < mend ? (x_row ? x_row[m0 + tid] : m0 + tid) : -1;
    const uint8_t* wrow[T::W_PT];
#pragma unroll
    for (int i = 0; i < T::W_PT; i++) {
        int n = n0 + (tid + i * T::NT) / 9;
        n = n < N ? n : N - 1;  // tail columns re-read a valid block; their outputs are dropped
        wrow[i] = n < n_split ? W1 + (size_t)n * row_bytes : W2 + (size_t)(n - n_split) * row_bytes;
    }

    float facc[RT][CT][4];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) facc[r][c][i] = 0.0f;

    uint4 ra[T::A_PT], rw[T::W_PT];
    float rdx;
    if (b0 < b1) mmq_fetch<RT, CT, WM, WN>(act, K, b0, tid, arow, wrow, dxrow, ra, rw, rdx);

    for (int b = b0; b < b1; b++) {
        __syncthreads();  // the previous superblock's LDS reads are done
        mmq_stage<RT, CT, WM, WN>(s_a, s_w, s_dx, tid, ra, rw, rdx);
        __syncthreads();
        if (b + 1 < b1) mmq_fetch<RT, CT, WM, WN>(act, K, b + 1, tid, arow, wrow, dxrow, ra, rw, rdx);

        v4i ia[RT][CT], ib[RT][CT], im[RT][CT];
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int c = 0; c < CT; c++) {
                ia[r][c] = v4i{0, 0, 0, 0};
                ib[r][c] = v4i{0, 0, 0, 0};
                im[r][c] = v4i{0, 0, 0, 0};
            }

        // per column tile: this lane's column header -> scale / min bytes
        uint32_t scw[CT][2], mnw[CT][2];
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const uint8_t* blk = s_w + (wn * CT * 16 + c * 16 + l16) * Q4K_BYTES;
            const uint4 hd = *reinterpret_cast<const uint4*>(blk);
            scw[c][0] = hd.y & 0x3f3f3f3fu;                                             // scales 0..3
            scw[c][1] = (hd.w & 0x0f0f0f0fu) | (((hd.y >> 6) & 0x03030303u) << 4);      // scales 4..7
            mnw[c][0] = hd.z & 0x3f3f3f3fu;                                             // mins 0..3
            mnw[c][1] = ((hd.w >> 4) & 0x0f0f0f0fu) | (((hd.z >> 6) & 0x03030303u) << 4);  // mins 4..7
        }

#pragma unroll
        for (int t = 0; t < 4; t++) {  // K steps of 64: sub-blocks 2t (kb < 2) and 2t+1 (kb >= 2)
            const int j = 2 * t + (kb >> 1);
            v4i afr[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const int8_t* pa = s_a + (wm * RT * 16 + r * 16 + l16) * A_STRIDE + 64 * t + 16 * kb;
                afr[r] = *reinterpret_cast<const v4i*>(pa);
            }
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const uint8_t* blk = s_w + (wn * CT * 16 + c * 16 + l16) * Q4K_BYTES;
                // element 64t + 16kb + i lives in qs[32t + 16(kb&1) + i], nibble kb>>1
                const uint4 raw = *reinterpret_cast<const uint4*>(blk + 16 + 32 * t + 16 * (kb & 1));
                const uint32_t sh = 4u * (uint32_t)(kb >> 1);
                // sub-block j = 2t + (kb>>1) sits in word t>>1 (compile-time), byte j&3
                const uint32_t jsh = 8u * (uint32_t)(j & 3);
                const uint32_t sc = (scw[c][t >> 1] >> jsh) & 0xffu;
                const uint32_t mn = (mnw[c][t >> 1] >> jsh) & 0xffu;
                const uint32_t a = sc >> 3, bb = sc & 7u;
                const uint32_t q0 = (raw.x >> sh) & 0x0f0f0f0fu, q1 = (raw.y >> sh) & 0x0f0f0f0fu;
                const uint32_t q2 = (raw.z >> sh) & 0x0f0f0f0fu, q3 = (raw.w >> sh) & 0x0f0f0f0fu;
                const v4i ba = v4i{(int)(q0 * a), (int)(q1 * a), (int)(q2 * a), (int)(q3 * a)};
                const v4i bbv = v4i{(int)(q0 * bb), (int)(q1 * bb), (int)(q2 * bb), (int)(q3 * bb)};
                const int mb = (int)(mn * 0x01010101u);
                const v4i bm = v4i{mb, mb, mb, mb};
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    ia[r][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], ba, ia[r][c], 0, 0, 0);
                    ib[r][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], bbv, ib[r][c], 0, 0, 0);
                    im[r][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], bm, im[r][c], 0, 0, 0);
                }
            }
        }

        // ---- f32 step: y += d_w*d_x*isum - dmin_w*d_x*msum ----
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const uint8_t* blk = s_w + (wn * CT * 16 + c * 16 + l16) * Q4K_BYTES;
            const uint32_t dd = *reinterpret_cast<const uint32_t*>(blk);
            const float dw = f16_to_f32(dd & 0xffffu), dmw = f16_to_f32(dd >> 16);
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float dx = s_dx[wm * RT * 16 + r * 16 + 4 * kb + i];
                    const int isum = 8 * ia[r][c][i] + ib[r][c][i];
                    facc[r][c][i] = fmaf(dw * dx, (float)isum, facc[r][c][i]);
                    facc[r][c][i] = fmaf(-(dmw * dx), (float)im[r][c][i], facc[r][c][i]);
                }
        }
    }

    float* out = nsplit > 1 ? y + (size_t)blockIdx.z * M * N : y;  // split partials: [z][M][N]
    const int ld = nsplit > 1 ? N : ldy;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int n = n0 + wn * CT * 16 + c * 16 + l16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + wm * RT * 16 + r * 16 + 4 * kb + i;
                if (m < mend && n < N) out[(size_t)m * ld + n] = facc[r][c][i];
            }
        }
}

// y[m][n] = sum over splits z (in order) of part[z][m][n]
__global__ void mmq_reduce_kernel(const float* __restrict__ part, float* __restrict__ y, int M, int N, int ldy,
                                  int nsplit) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * N) return;
    float s = part[i];
    for (int z = 1; z < nsplit; z++) s += part[(size_t)z * M * N + i];
    y[(i / N) * ldy + i % N] = s;
}

template <int RT, int CT, int WM, int WN>
hipError_t launch_cfg(const uint8_t* w, ActView act, float* y, float* part, size_t part_elems, int M, int N, int K,
                      int ldy, int num_cus, hipStream_t s) {
    using T = MmqTile<RT, CT, WM, WN>;
    const int mt = (M + T::BM - 1) / T::BM, nt = (N + T::BN - 1) / T::BN;
    const int KB = K / QK_K;
    // split K when the tile grid cannot fill two workgroups per CU, keeping >= 2 superblocks per split
    int ks = 1;
    const int tiles = mt * nt;
    if (part && tiles < 2 * num_cus) {
        ks = (2 * num_cus + tiles - 1) / tiles;
        const int kmax = KB / 2 > 1 ? KB / 2 : 1;
        if (ks > kmax) ks = kmax;
        while (ks > 1 && (size_t)ks * M * N > part_elems) ks--;
    }
    dim3 grid(mt, nt, ks);
    hipLaunchKernelGGL((mmq_q4k_kernel<RT, CT, WM, WN, false>), grid, dim3(T::NT), 0, s, w, act, ks > 1 ? part : y,
                       M, N, K, ldy, MmqGroup{});
    if (ks > 1) {
        const size_t total = (size_t)M * N;
        hipLaunchKernelGGL(mmq_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, y, M, N,
                           ldy, ks);
    }
    return hipGetLastError();
}

template <int RT, int CT, int WM, int WN>
hipError_t launch_grouped_cfg(const uint8_t* w, ActView act, float* y, int max_tiles, int N, int K, int ldy,
                              const MmqGroup& g, hipStream_t s) {
    using T = MmqTile<RT, CT, WM, WN>;
    dim3 grid(max_tiles, (N + T::BN - 1) / T::BN, 1);
    hipLaunchKernelGGL((mmq_q4k_kernel<RT, CT, WM, WN, true>), grid, dim3(T::NT), 0, s, w, act, y, 0, N, K, ldy, g);
    return hipGetLastError();
}

}  // namespace

int mmq_group_rows(int rows_per_expert) { return rows_per_expert >= 24 ? 32 : 16; }

hipError_t launch_mmq_grouped(int dtype, const uint8_t* w, ActView act, float* y, int bm, int max_tiles, int N, int K,
                              int ldy, const MmqGroup& g, hipStream_t s) {
    if (dtype != GGML_Q4K || max_tiles <= 0) return max_tiles == 0 ? hipSuccess : hipErrorInvalidValue;
    if (bm == 32) return launch_grouped_cfg<2, 1, 1, 4>(w, act, y, max_tiles, N, K, ldy, g, s);  // 32 x 64
    if (bm == 16) return launch_grouped_cfg<1, 1, 1, 4>(w, act, y, max_tiles, N, K, ldy, g, s);  // 16 x 64
    return hipErrorInvalidValue;
}

bool mmq_supported(int dtype) { return dtype == GGML_Q4K; }

size_t mmq_partial_elems(int M, int N, int num_cus) {
    // enough split partials for the widest split launch_cfg picks (2 x CUs tiles)
    return (size_t)M * N * (size_t)(2 * num_cus > 64 ? 64 : 2 * num_cus);
}

hipError_t launch_mmq(int dtype, const uint8_t* w, ActView act, float* y, float* part, size_t part_elems, int M,
                      int N, int K, int ldy, int num_cus, hipStream_t s) {
    if (dtype != GGML_Q4K) return hipErrorInvalidValue;
    if (M >= 128) return launch_cfg<4, 2, 2, 2>(w, act, y, part, part_elems, M, N, K, ldy, num_cus, s);  // 128 x 64
    if (M >= 64) return launch_cfg<2, 2, 2, 2>(w, act, y, part, part_elems, M, N, K, ldy, num_cus, s);   // 64 x 64
    return launch_cfg<2, 1, 1, 4>(w, act, y, part, part_elems, M, N, K, ldy, num_cus, s);                // 32 x 64
}

}  // namespace frq
