// Batched / prefill quantized matmul (M >= 16) on gfx950 int8 MFMA:
// fuel's matmul<BlockQ4K> and matmul<BlockQ6K> (k_quants.rs:2284-2331) for
// many activation rows, with the same per-superblock integer sums as the
// scalar vec_dots (k_quants.rs:1388-1468, 1946-2003) and one f32 step per
// superblock.  Activations are Q8K rows (one int8 per element, one f32 scale
// per 256), quantized once per call.
//
// Q4_K.  Per superblock, with q4 the weight nibbles, sc_j / m_j the 6-bit
// scale / min of sub-block j and q8 the activation:
//   isum = sum_j sc_j * sum_{e in j} q4_e q8_e ,  msum = sum_j m_j * S_j
// with S_j = sum_{e in j} q8_e.  A 6-bit scale times a nibble does not fit
// int8, so sc_j = 8*a_j + b_j with a_j, b_j <= 7: q4*a_j and q4*b_j are <= 105
// and fit a byte.  Then
//   isum = 8 * (X . Ba) + (X . Bb),   msum = X . Bm
// with Bm the sub-block mins broadcast over their 32 elements: three int8
// GEMMs over K = 256 per superblock, exact in int32.  (The kernel is bound by
// its VALU work, not the matrix cores: msum on the MFMA pipe costs less than
// its 8-term dot products on the VALU.)  f32 step: y += d_x*(d*isum - dmin*msum).
//
// Q6_K.  w_e = (q6_e - 32) * sc_g, with sc_g the int8 scale of 16-element
// group g, lies in [-4096, 4064]: split w = 128*wh + wl with wl = w & 127 in
// [0, 127] and wh = w >> 7 (arithmetic) in [-32, 31], both bytes, so
//   isum = 128 * (X . Wh) + (X . Wl)
// is two exact int8 GEMMs.  The products are formed two per 16-bit lane with
// one packed multiply-add.  f32 step: y += d_x * (d * isum).
//
// Workgroup: WM x WN wavefronts, each owning RT x CT tiles of 16x16 outputs.
// Per superblock the workgroup stages the quantized activation rows (272-byte
// LDS row stride), their scales and the raw weight blocks of its columns in
// LDS, double-buffered: the next superblock's global loads are in
// flight while the current one is multiplied, and one barrier per superblock
// separates the two buffers' roles.  Lanes build their B fragments in
// registers from the raw blocks.
#include <type_traits>
#include <utility>

#include "common.hpp"
#include "kernels.hpp"
#include "mfma.hpp"

namespace frq {

namespace {

constexpr int A_STRIDE = QK_K + 16;  // LDS bytes per activation row per superblock

// ---- format policies ----
// CH 16-byte chunks are staged per column and superblock: chunk ch comes from
// global byte src(ch) of the block and lands at LDS byte 16*ch of the
// column's STRIDE-byte slot.

struct MmqQ4K {
    static constexpr int BYTES = Q4K_BYTES, STRIDE = Q4K_BYTES, CH = 9, NACC = 3;
    __device__ static uint32_t src(int ch) { return 16u * (uint32_t)ch; }
    struct Hdr {
        uint32_t sc[2], mn[2];  // 6-bit scales / mins of sub-blocks 0..3, 4..7 (one byte each)
        float d, dmin;
    };
    __device__ static void header(const uint8_t* col, Hdr& h) {
        const uint4 hd = *reinterpret_cast<const uint4*>(col);
        h.sc[0] = hd.y & 0x3f3f3f3fu;
        h.sc[1] = (hd.w & 0x0f0f0f0fu) | (((hd.y >> 6) & 0x03030303u) << 4);
        h.mn[0] = hd.z & 0x3f3f3f3fu;
        h.mn[1] = ((hd.w >> 4) & 0x0f0f0f0fu) | (((hd.z >> 6) & 0x03030303u) << 4);
        h.d = f16_to_f32(hd.x & 0xffffu);
        h.dmin = f16_to_f32(hd.x >> 16);
    }
    // K step t (elements 64t..64t+63): lane group kb holds elements 64t+16kb+[0,16).
    template <int RT, int CT>
    __device__ static void step(int t, int kb, int c, const uint8_t* col, const Hdr& h, const v4i (&afr)[RT],
                                v4i (&acc)[RT][CT][NACC]) {
        // element 64t + 16kb + i lives in qs[32t + 16(kb&1) + i], nibble kb>>1
        const uint4 raw = *reinterpret_cast<const uint4*>(col + 16 + 32 * t + 16 * (kb & 1));
        const uint32_t sh = 4u * (uint32_t)(kb >> 1);
        // sub-block j = 2t + (kb>>1) sits in word t>>1 (compile-time), byte j&3
        const uint32_t jsh = 8u * (uint32_t)((2 * t + (kb >> 1)) & 3);
        const uint32_t sc = (h.sc[t >> 1] >> jsh) & 0xffu;
        const uint32_t mn = (h.mn[t >> 1] >> jsh) & 0xffu;
        const uint32_t a = sc >> 3, bb = sc & 7u;
        const uint32_t q0 = (raw.x >> sh) & 0x0f0f0f0fu, q1 = (raw.y >> sh) & 0x0f0f0f0fu;
        const uint32_t q2 = (raw.z >> sh) & 0x0f0f0f0fu, q3 = (raw.w >> sh) & 0x0f0f0f0fu;
        const v4i ba = v4i{bytes_times(q0, a), bytes_times(q1, a), bytes_times(q2, a), bytes_times(q3, a)};
        const v4i bbv = v4i{bytes_times(q0, bb), bytes_times(q1, bb), bytes_times(q2, bb), bytes_times(q3, bb)};
        const int mb = (int)(__builtin_amdgcn_perm(0u, mn, 0x00000000u));  // the byte in all four lanes
        const v4i bm = v4i{mb, mb, mb, mb};
        const v4i zero = v4i{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < RT; r++) {
            acc[r][c][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], ba, t == 0 ? zero : acc[r][c][0], 0, 0, 0);
            acc[r][c][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], bbv, t == 0 ? zero : acc[r][c][1], 0, 0, 0);
            acc[r][c][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], bm, t == 0 ? zero : acc[r][c][2], 0, 0, 0);
        }
    }
    // d*isum - dmin*msum of output element i of the lane's 16x16 tile
    __device__ static float finish(const v4i (&a)[NACC], int i, const Hdr& h) {
        const int isum = 8 * a[0][i] + a[1][i];
        return fmaf(-h.dmin, (float)a[2][i], h.d * (float)isum);
    }
};

struct MmqQ6K {
    // 210-byte blocks sit at 2-byte alignment: chunks 0..12 are bytes
    // 0..207 (ql, qh, scales) and chunk 13 is bytes 194..209, which puts d at
    // LDS byte 222 and never reads past the block.
    static constexpr int BYTES = Q6K_BYTES, STRIDE = 224, CH = 14, NACC = 2;
    __device__ static uint32_t src(int ch) { return ch < 13 ? 16u * (uint32_t)ch : 194u; }
    struct Hdr {
        uint32_t sc[4];  // int8 scales 4t..4t+3 in word t
        float d;
    };
    __device__ static void header(const uint8_t* col, Hdr& h) {
        const uint4 s = *reinterpret_cast<const uint4*>(col + 192);
        h.sc[0] = s.x;
        h.sc[1] = s.y;
        h.sc[2] = s.z;
        h.sc[3] = s.w;
        h.d = f16_to_f32(*reinterpret_cast<const uint16_t*>(col + 222));
    }
    // Element 64t + 16kb + i is element 128hh + 32qd + l of fuel's layout
    // (k_quants.rs:2170-2186) with hh = t>>1, qd = 2(t&1) + (kb>>1),
    // l = 16(kb&1) + i: low (t even) / high (t odd) nibble of
    // ql[64hh + 32(kb>>1) + l] and bits 2qd..2qd+1 of qh[32hh + l]; its scale
    // is scales[4t + kb].
    template <int RT, int CT>
    __device__ static void step(int t, int kb, int c, const uint8_t* col, const Hdr& h, const v4i (&afr)[RT],
                                v4i (&acc)[RT][CT][NACC]) {
        const uint4 ql = *reinterpret_cast<const uint4*>(col + 64 * (t >> 1) + 32 * (kb >> 1) + 16 * (kb & 1));
        const uint4 qh = *reinterpret_cast<const uint4*>(col + 128 + 32 * (t >> 1) + 16 * (kb & 1));
        const uint32_t ls = 4u * (uint32_t)(t & 1);                   // compile-time
        const uint32_t hs = 4u * (uint32_t)(t & 1) + 2u * (uint32_t)(kb >> 1);
        const int sc = (int)(int8_t)((h.sc[t] >> (8 * kb)) & 0xffu);
        const uint32_t f = (uint32_t)sc & 0xffffu, cst = (uint32_t)(-32 * sc) & 0xffffu;
        const uint32_t sc16 = f | (f << 16), c16 = cst | (cst << 16);
        const uint32_t l4[4] = {ql.x, ql.y, ql.z, ql.w}, h4[4] = {qh.x, qh.y, qh.z, qh.w};
        int wl[4], wh[4];
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t u = ((l4[d] >> ls) & 0x0f0f0f0fu) | (((h4[d] >> hs) & 0x03030303u) << 4);
            q6_planes(u, sc16, c16, wl[d], wh[d]);
        }
        const v4i bh = v4i{wh[0], wh[1], wh[2], wh[3]}, bl = v4i{wl[0], wl[1], wl[2], wl[3]};
        const v4i zero = v4i{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < RT; r++) {
            acc[r][c][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], bh, t == 0 ? zero : acc[r][c][0], 0, 0, 0);
            acc[r][c][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], bl, t == 0 ? zero : acc[r][c][1], 0, 0, 0);
        }
    }
    __device__ static float finish(const v4i (&a)[NACC], int i, const Hdr& h) {
        const int isum = 128 * a[0][i] + a[1][i];
        return h.d * (float)isum;
    }
};

template <class F, int RT, int CT, int WM, int WN>
struct MmqTile {
    static constexpr int NT = 64 * WM * WN;
    static constexpr int BM = 16 * RT * WM, BN = 16 * CT * WN;
    static constexpr int A_CH = BM * 16;     // 16-byte activation chunks per superblock
    static constexpr int W_CH = BN * F::CH;  // 16-byte weight chunks per superblock
    static constexpr int A_PT = (A_CH + NT - 1) / NT;
    static constexpr int W_PT = (W_CH + NT - 1) / NT;
    // LDS per buffer: activations, weights, activation scales
    static constexpr int LDS_A = BM * A_STRIDE, LDS_W = BN * F::STRIDE, LDS_D = BM * 4;
    static constexpr int LDS_BUF = LDS_A + LDS_W + LDS_D;
};

// Register copy of one superblock's share of a thread: activation chunks,
// weight chunks, one activation scale.
template <class F, int RT, int CT, int WM, int WN>
struct MmqRegs {
    using T = MmqTile<F, RT, CT, WM, WN>;
    uint4 a[T::A_PT], w[T::W_PT];
    float dx;
};

// Global loads of superblock b: 32-bit per-lane offsets from uniform base
// pointers (the SGPR-base addressing form: no 64-bit address arithmetic per
// load).  aoff < 0 marks a padding row (staged as zeros).
template <class F, int RT, int CT, int WM, int WN>
__device__ __forceinline__ void mmq_fetch(const int8_t* __restrict__ qs, const float* __restrict__ dv,
                                          const uint8_t* __restrict__ wbase, int b, int tid,
                                          const int (&aoff)[MmqTile<F, RT, CT, WM, WN>::A_PT],
                                          const uint32_t (&woff)[MmqTile<F, RT, CT, WM, WN>::W_PT], int dxoff,
                                          MmqRegs<F, RT, CT, WM, WN>& g) {
    using T = MmqTile<F, RT, CT, WM, WN>;
    const uint32_t ab = (uint32_t)b * QK_K, wb = (uint32_t)b * F::BYTES;
#pragma unroll
    for (int i = 0; i < T::A_PT; i++) {
        g.a[i] = uint4{0u, 0u, 0u, 0u};  // (set on every path: a conditionally-set array lives in scratch)
        if (aoff[i] >= 0) g.a[i] = *reinterpret_cast<const uint4*>(qs + ((uint32_t)aoff[i] + ab));
    }
#pragma unroll
    for (int i = 0; i < T::W_PT; i++) {
        g.w[i] = uint4{0u, 0u, 0u, 0u};
        if (tid + i * T::NT < T::W_CH) g.w[i] = load16_u(wbase + (woff[i] + wb));
    }
    g.dx = dxoff >= 0 ? dv[(uint32_t)dxoff + (uint32_t)b] : 0.0f;
}

// Registers -> LDS buffer.
template <class F, int RT, int CT, int WM, int WN>
__device__ __forceinline__ void mmq_stage(uint8_t* buf, int tid, const MmqRegs<F, RT, CT, WM, WN>& g) {
    using T = MmqTile<F, RT, CT, WM, WN>;
    int8_t* s_a = reinterpret_cast<int8_t*>(buf);
    uint8_t* s_w = buf + T::LDS_A;
    float* s_d = reinterpret_cast<float*>(buf + T::LDS_A + T::LDS_W);
#pragma unroll
    for (int i = 0; i < T::A_PT; i++) {
        const int idx = tid + i * T::NT;
        if (idx < T::A_CH) *reinterpret_cast<uint4*>(s_a + (idx >> 4) * A_STRIDE + 16 * (idx & 15)) = g.a[i];
    }
#pragma unroll
    for (int i = 0; i < T::W_PT; i++) {
        const int idx = tid + i * T::NT;
        if (idx < T::W_CH) *reinterpret_cast<uint4*>(s_w + (idx / F::CH) * F::STRIDE + 16 * (idx % F::CH)) = g.w[i];
    }
    if (tid < T::BM) s_d[tid] = g.dx;
}

// grid: non-grouped, a 1-D list of (M tile, N tile, K split) tiles in an
// XCD-aware order (consecutive workgroups go to different XCDs on MI355X, so
// tile t of XCD x is x's own contiguous range: the M tiles sharing a weight
// tile share that XCD's L2).  With ksplit > 1 each workgroup sums a contiguous
// range of superblocks into part[split][M][N]; mmq_reduce_kernel adds the
// splits in order afterwards (deterministic).
// GROUPED (MoE): grid (tile table bound, N tiles); workgroup x takes tile x of
// the expert-sorted rows (g.tile_*); its rows end at its expert's end offset,
// its weights are that expert's, and activation row m is g.x_row[m] (gathered
// token rows) when x_row is set.
template <class F, int RT, int CT, int WM, int WN, bool GROUPED>
__global__ __launch_bounds__(64 * WM * WN) void mmq_kernel(const uint8_t* __restrict__ W, ActView act,
                                                           float* __restrict__ y, int M, int N, int K, int ldy,
                                                           int mt, int nt, int nsplit, int out_mode, MmqGroup g) {
    using T = MmqTile<F, RT, CT, WM, WN>;
    constexpr int BM = T::BM, BN = T::BN;
    __shared__ __align__(16) uint8_t smem[2 * T::LDS_BUF];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int KB = K / QK_K;
    const size_t row_bytes = (size_t)KB * F::BYTES;
    const int l16 = lane & 15, kb = lane >> 4;

    int mtile, ntile, split;
    if constexpr (GROUPED) {
        mtile = blockIdx.x;
        ntile = blockIdx.y;
        split = 0;
    } else {
        const int total = mt * nt * nsplit, L = blockIdx.x;
        const int x = L & 7, slot = L >> 3, q = total >> 3, r = total & 7;
        const int t = x * q + (x < r ? x : r) + slot;  // XCD x's contiguous range of tiles
        mtile = t % mt;
        ntile = (t / mt) % nt;
        split = t / (mt * nt);
    }
    const int b0 = (int)((long long)KB * split / nsplit), b1 = (int)((long long)KB * (split + 1) / nsplit);
    const int n0 = ntile * BN;
    int m0 = mtile * BM, mend = M, n_split = N;
    const uint8_t* W1 = W;
    const uint8_t* W2 = W;
    const int* x_row = nullptr;
    if constexpr (GROUPED) {
        if (mtile >= *g.ntiles) return;  // uniform: the tile table is shorter than the grid bound
        const int e = g.tile_expert[mtile];
        m0 = g.tile_row0[mtile];
        mend = g.expert_offsets[e + 1];
        W1 = W + (size_t)e * g.expert_bytes;
        W2 = g.w2 ? g.w2 + (size_t)e * g.expert_bytes : W1;
        if (g.w2) n_split = g.n_split;
        x_row = g.x_row;
    }
    // per-thread byte offsets of each staged chunk in superblock 0 (-1: padding row)
    int aoff[T::A_PT];
#pragma unroll
    for (int i = 0; i < T::A_PT; i++) {
        const int idx = tid + i * T::NT;
        const int m = m0 + (idx >> 4);
        aoff[i] = idx < T::A_CH && m < mend ? (x_row ? x_row[m] : m) * K + 16 * (idx & 15) : -1;
    }
    const int dxoff = tid < BM && m0 + tid < mend ? (x_row ? x_row[m0 + tid] : m0 + tid) * KB : -1;
    // the workgroup's columns lie on one side of n_split (a multiple of BN)
    const bool second = n0 >= n_split;
    const uint8_t* wbase = second ? W2 : W1;
    uint32_t woff[T::W_PT];
#pragma unroll
    for (int i = 0; i < T::W_PT; i++) {
        const int idx = tid + i * T::NT;
        int n = n0 + idx / F::CH;
        n = n < N ? n : N - 1;  // tail columns re-read a valid block; their outputs are dropped
        woff[i] = (uint32_t)(second ? n - n_split : n) * (uint32_t)row_bytes + F::src(idx % F::CH);
    }

    float facc[RT][CT][4];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) facc[r][c][i] = 0.0f;

    MmqRegs<F, RT, CT, WM, WN> regs;
    if (b0 < b1) {
        mmq_fetch<F, RT, CT, WM, WN>(act.qs, act.d, wbase, b0, tid, aoff, woff, dxoff, regs);
        mmq_stage<F, RT, CT, WM, WN>(smem, tid, regs);
    }
    __syncthreads();

    for (int b = b0; b < b1; b++) {
        uint8_t* buf = smem + ((b - b0) & 1) * T::LDS_BUF;
        const bool more = b + 1 < b1;
        if (more) mmq_fetch<F, RT, CT, WM, WN>(act.qs, act.d, wbase, b + 1, tid, aoff, woff, dxoff, regs);
        const int8_t* s_a = reinterpret_cast<const int8_t*>(buf);
        const uint8_t* s_w = buf + T::LDS_A;
        const float* s_d = reinterpret_cast<const float*>(buf + T::LDS_A + T::LDS_W);

        v4i acc[RT][CT][F::NACC];  // set by the first K step (zero accumulator input)
        typename F::Hdr hdr[CT];   // per column tile: this lane's column header
#pragma unroll
        for (int c = 0; c < CT; c++) F::header(s_w + (wn * CT * 16 + c * 16 + l16) * F::STRIDE, hdr[c]);

#pragma unroll
        for (int t = 0; t < 4; t++) {  // K steps of 64
            v4i afr[RT];
#pragma unroll
            for (int r = 0; r < RT; r++)
                afr[r] = *reinterpret_cast<const v4i*>(s_a + (wm * RT * 16 + r * 16 + l16) * A_STRIDE + 64 * t +
                                                       16 * kb);
#pragma unroll
            for (int c = 0; c < CT; c++)
                F::template step<RT, CT>(t, kb, c, s_w + (wn * CT * 16 + c * 16 + l16) * F::STRIDE, hdr[c], afr, acc);
        }

        // ---- f32 step per superblock ----
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float dx = s_d[wm * RT * 16 + r * 16 + 4 * kb + i];
#pragma unroll
                for (int c = 0; c < CT; c++) facc[r][c][i] = fmaf(dx, F::finish(acc[r][c], i, hdr[c]), facc[r][c][i]);
            }
        if (more) mmq_stage<F, RT, CT, WM, WN>(smem + ((b + 1 - b0) & 1) * T::LDS_BUF, tid, regs);
        __syncthreads();
    }

    float* out = nsplit > 1 ? y + (size_t)split * M * N : y;  // split partials: [z][M][N]
    const int ld = nsplit > 1 ? N : ldy;
    const int omode = nsplit == 1 ? out_mode : 0;  // (split partials: plain f32; the reduce applies the mode)
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int n = n0 + wn * CT * 16 + c * 16 + l16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + wm * RT * 16 + r * 16 + 4 * kb + i;
                if (m < mend && n < N) store_out(out, (size_t)m * ld + n, facc[r][c][i], omode);
            }
        }
}

// ---- Q4_K with the staging through LDS DMA ----
// The same tile computation, but every superblock's activation rows, weight
// blocks and activation scales go global -> LDS with global_load_lds (each
// lane's 16 or 4 bytes land at the instruction's LDS base + lane * size), into
// a ring of three LDS buffers: superblock b+2 is in flight while b is
// multiplied, with no staging registers and no LDS stores.  The waits are
// explicit: before superblock b is read, each wavefront lets only b+1's loads
// stay outstanding (s_waitcnt vmcnt), then one barrier per superblock.  The
// three buffers are distinct LDS objects and the loop is unrolled by three,
// so the compiler sees which buffer each load writes and adds no waits of its
// own.  Activation rows are stored 256 bytes apart with chunk j of row r at
// position j ^ (r & 15): the 16 rows an MFMA fragment read touches fall in
// different banks.  Needs 16-byte aligned weight blocks (Q4_K: 144 bytes).

#define FRQ_VMCNT(n) ((((n) & 0xF) | (((n) >> 4) << 14) | (7 << 4) | (0xF << 8)))

template <class F, int RT, int CT, int WM, int WN>
struct DmaTile {
    static constexpr int NW = WM * WN, NT = 64 * NW;
    static constexpr int BM = 16 * RT * WM, BN = 16 * CT * WN;
    static constexpr int A_INST = BM / 4;  // 16 chunks per row, 64 per instruction
    static_assert(A_INST % NW == 0, "activation tile must split evenly over the wavefronts");
    static constexpr int A_PW = A_INST / NW;
    static constexpr int W_CH = BN * F::CH;
    static constexpr int W_INST = (W_CH + 63) / 64;
    static constexpr int W_PW = (W_INST + NW - 1) / NW;
    static constexpr int D_PW = ((BM + 63) / 64 + NW - 1) / NW;
    static constexpr int NI = A_PW + W_PW + D_PW;  // load instructions per wavefront and superblock
    static_assert(NI <= 63, "vmcnt range");
    static constexpr int LA = A_PW * NW * 1024, LW = W_PW * NW * 1024, LD = D_PW * NW * 64;
};

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// (kept in device functions: the builtin may not appear in a kernel body the
// host pass instantiates)
__device__ __forceinline__ void lds_dma16(const uint8_t* g, uint8_t* l) { __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0); }
__device__ __forceinline__ void lds_dma4(const uint8_t* g, uint8_t* l) { __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0); }

template <class F, int RT, int CT, int WM, int WN, bool GROUPED>
__global__ __launch_bounds__(64 * WM * WN) void mmq_dma_kernel(const uint8_t* __restrict__ W, ActView act,
                                                               float* __restrict__ y, int M, int N, int K, int ldy,
                                                               int mt, int nt, int nsplit, int out_mode, MmqGroup g) {
    using T = DmaTile<F, RT, CT, WM, WN>;
    constexpr int BM = T::BM, BN = T::BN, NW = T::NW;
    __shared__ __align__(16) uint8_t sA0[T::LA], sA1[T::LA], sA2[T::LA];
    __shared__ __align__(16) uint8_t sW0[T::LW], sW1[T::LW], sW2[T::LW];
    __shared__ __align__(16) float sD0[T::LD], sD1[T::LD], sD2[T::LD];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int KB = K / QK_K;
    const uint32_t row_bytes = (uint32_t)KB * F::BYTES;
    const int l16 = lane & 15, kb = lane >> 4;

    int mtile, ntile, split;
    if constexpr (GROUPED) {
        mtile = blockIdx.x;
        ntile = blockIdx.y;
        split = 0;
    } else {
        const int total = mt * nt * nsplit, L = blockIdx.x;
        const int x = L & 7, slot = L >> 3, q = total >> 3, r = total & 7;
        const int t = x * q + (x < r ? x : r) + slot;  // XCD x's contiguous range of tiles
        mtile = t % mt;
        ntile = (t / mt) % nt;
        split = t / (mt * nt);
    }
    const int b0 = (int)((long long)KB * split / nsplit), b1 = (int)((long long)KB * (split + 1) / nsplit);
    const int n0 = ntile * BN;
    int m0 = mtile * BM, mend = M, n_split = N;
    const uint8_t* W1 = W;
    const uint8_t* W2 = W;
    const int* x_row = nullptr;
    if constexpr (GROUPED) {
        if (mtile >= *g.ntiles) return;  // uniform: the tile table is shorter than the grid bound
        const int e = g.tile_expert[mtile];
        m0 = g.tile_row0[mtile];
        mend = g.expert_offsets[e + 1];
        W1 = W + (size_t)e * g.expert_bytes;
        W2 = g.w2 ? g.w2 + (size_t)e * g.expert_bytes : W1;
        if (g.w2) n_split = g.n_split;
        x_row = g.x_row;
    }
    const bool second = n0 >= n_split;  // the workgroup's columns lie on one side of n_split
    const uint8_t* wbase = second ? W2 : W1;
    const uint8_t* dbase = reinterpret_cast<const uint8_t*>(act.d);
    const uint8_t* qbase = reinterpret_cast<const uint8_t*>(act.qs);

    // per-lane source byte offsets of superblock 0 (padding slots read offset 0,
    // a valid address; their LDS bytes are never used)
    uint32_t asrc[T::A_PW], wsrc[T::W_PW], dsrc[T::D_PW];
#pragma unroll
    for (int j = 0; j < T::A_PW; j++) {
        const int q = 64 * (j * NW + wave) + lane, r = q >> 4, m = m0 + r;
        const int row = m < mend ? (x_row ? x_row[m] : m) : 0;
        asrc[j] = (uint32_t)row * (uint32_t)K + 16u * (uint32_t)((q & 15) ^ (r & 15));
    }
#pragma unroll
    for (int j = 0; j < T::W_PW; j++) {
        const int q = 64 * (j * NW + wave) + lane;
        int n = n0 + q / F::CH;
        n = n < N ? n : N - 1;  // tail columns re-read a valid block; their outputs are dropped
        wsrc[j] = q < T::W_CH ? (uint32_t)(second ? n - n_split : n) * row_bytes + F::src(q % F::CH) : 0u;
    }
#pragma unroll
    for (int j = 0; j < T::D_PW; j++) {
        const int q = 64 * (j * NW + wave) + lane, m = m0 + q;
        dsrc[j] = q < BM && m < mend ? 4u * (uint32_t)((x_row ? x_row[m] : m) * KB) : 0u;
    }

    auto issue = [&](int b, uint8_t* A, uint8_t* Wd, float* D) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < T::A_PW; j++) lds_dma16(qbase + (asrc[j] + (uint32_t)b * QK_K), A + 1024 * (j * NW + wave));
#pragma unroll
        for (int j = 0; j < T::W_PW; j++)
            lds_dma16(wbase + (wsrc[j] + (uint32_t)b * F::BYTES), Wd + 1024 * (j * NW + wave));
#pragma unroll
        for (int j = 0; j < T::D_PW; j++)
            lds_dma4(dbase + (dsrc[j] + 4u * (uint32_t)b), reinterpret_cast<uint8_t*>(D) + 256 * (j * NW + wave));
    };

    float facc[RT][CT][4];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) facc[r][c][i] = 0.0f;

    if (b0 < b1) issue(b0, sA0, sW0, sD0);
    if (b0 + 1 < b1) issue(b0 + 1, sA1, sW1, sD1);

    auto iter = [&](auto kr, int b) __attribute__((always_inline)) {
        constexpr int KR = decltype(kr)::value;
        uint8_t* A = KR == 0 ? sA0 : KR == 1 ? sA1 : sA2;
        uint8_t* Wd = KR == 0 ? sW0 : KR == 1 ? sW1 : sW2;
        float* D = KR == 0 ? sD0 : KR == 1 ? sD1 : sD2;
        // superblock b landed (only b+1's loads may stay in flight), in every wavefront
        if (b + 1 < b1) __builtin_amdgcn_s_waitcnt(FRQ_VMCNT(T::NI));
        else __builtin_amdgcn_s_waitcnt(FRQ_VMCNT(0));
        compiler_fence();
        __builtin_amdgcn_s_barrier();
        compiler_fence();
        // the buffer of b+2 was last read in iteration b-1, which every wavefront has left
        if (b + 2 < b1) {
            constexpr int KN = (KR + 2) % 3;
            issue(b + 2, KN == 0 ? sA0 : KN == 1 ? sA1 : sA2, KN == 0 ? sW0 : KN == 1 ? sW1 : sW2,
                  KN == 0 ? sD0 : KN == 1 ? sD1 : sD2);
        }
        v4i acc[RT][CT][F::NACC];  // set by the first K step (zero accumulator input)
        typename F::Hdr hdr[CT];
#pragma unroll
        for (int c = 0; c < CT; c++) F::header(Wd + (wn * CT * 16 + c * 16 + l16) * F::STRIDE, hdr[c]);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            v4i afr[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const int row = wm * RT * 16 + r * 16 + l16;  // row & 15 == l16
                afr[r] = *reinterpret_cast<const v4i*>(A + row * QK_K + 16 * ((4 * t + kb) ^ l16));
            }
#pragma unroll
            for (int c = 0; c < CT; c++)
                F::template step<RT, CT>(t, kb, c, Wd + (wn * CT * 16 + c * 16 + l16) * F::STRIDE, hdr[c], afr, acc);
        }
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float dx = D[wm * RT * 16 + r * 16 + 4 * kb + i];
#pragma unroll
                for (int c = 0; c < CT; c++) facc[r][c][i] = fmaf(dx, F::finish(acc[r][c], i, hdr[c]), facc[r][c][i]);
            }
    };
    for (int b = b0; b < b1; b += 3) {
        iter(std::integral_constant<int, 0>{}, b);
        if (b + 1 < b1) iter(std::integral_constant<int, 1>{}, b + 1);
        if (b + 2 < b1) iter(std::integral_constant<int, 2>{}, b + 2);
    }

    float* out = nsplit > 1 ? y + (size_t)split * M * N : y;  // split partials: [z][M][N]
    const int ld = nsplit > 1 ? N : ldy;
    const int omode = nsplit == 1 ? out_mode : 0;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int n = n0 + wn * CT * 16 + c * 16 + l16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + wm * RT * 16 + r * 16 + 4 * kb + i;
                if (m < mend && n < N) store_out(out, (size_t)m * ld + n, facc[r][c][i], omode);
            }
        }
}

// ---- Q4_K, wide tiles: two MFMAs per product ----
// NW wavefronts side by side in N share BM = 16 RT activation rows; each owns
// 16 CT weight columns, so every weight block is unpacked by one wavefront.
// Per superblock, one LDS ring slot receives, by DMA (global_load_lds, no
// staging registers, no LDS stores): the activation rows (256 bytes each,
// chunk j of row r at position j ^ (r & 15)), the raw weight blocks of the
// BN columns (144 bytes apart, in their byte order), the rows' 16-element
// sums (32 bytes a row) and their scales.  Two slots: superblock b+1 is in
// flight while b is multiplied (issued right after the barrier that ends
// everyone's reads of its slot); the DMA instructions of a slot are dealt out
// round-robin to the wavefronts, each issuing the same count (the spare ones
// repeat the slot's last activation load: same source, same bytes, same
// place).
//
// K order inside a superblock: K step t (64 elements) has lane group kb take
// the 16 elements of qs bytes 64 (t&1) + 16 kb .. +15, low nibbles for t < 2
// and high nibbles for t >= 2 (the shift is uniform per step).  In fuel's
// layout (k_quants.rs:1421-1440) qs byte i holds element 64 (i/32) + i%32 in
// its low nibble and that + 32 in its high one, so the lane's elements are
// 32 s + 16 (kb&1) + [0,16) of sub-block s = 4 (t&1) + 2 (kb>>1) + (t>>1):
// its scale is byte 2 (kb>>1) + (t>>1) of scale word t&1 and its activation
// chunk is 2 s + (kb&1).
//
// isum = 8 (X . Ba) + (X . Bb) as in MmqQ4K; msum = sum_j m_j S_j comes from
// one f16 MFMA per superblock, K = 16 over the activation's 16-element sums
// b_i (the quantizer's f16 copy: |b_i| <= 2032 is exact) against m_{i/2}
// (<= 63): every product and partial sum is an integer below 2^24, exact in
// the f32 accumulator.
// The f32 step is MmqQ4K's y += d_x * (d * isum - dmin * msum), the same
// operations in the same order.
typedef _Float16 wh4 __attribute__((ext_vector_type(4)));
typedef float wf4 __attribute__((ext_vector_type(4)));

// LDS DMA through inline assembly: the compiler does not see these loads, so
// it inserts no waits of its own for them (it cannot tell the ring slot being
// filled from the slot being read and would wait for every load in flight
// before the first read); the kernel's explicit waits are the only ones, and
// they are exact: before a slot is read, s_waitcnt vmcnt(0) and a barrier.
// The compiler's waits for its own loads stay safe, since vmcnt counts in
// issue order and hidden loads only make them wait longer.  M0 holds the LDS
// address of lane 0 (wave-uniform), lane i writes at M0 + i * size, with one
// wait state between the M0 write and the DMA.  Nothing else in the kernel
// that issues these uses M0 (no indirect register indexing, no LDS-DMA
// builtins, no messages), so the clobber the compiler cannot preserve loses
// nothing.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_asm(const uint8_t* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4_asm(const uint8_t* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

template <int... I, class Fn>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, Fn&& fn) {
    (fn(std::integral_constant<int, I>{}), ...);
}
// fn(integral_constant<int, i>) for i = 0 .. n-1
template <int n, class Fn>
__device__ __forceinline__ void static_for(Fn&& fn) {
    static_for_impl(std::make_integer_sequence<int, n>{}, fn);
}

template <int RT, int CT, int NW>
struct WideTile {
    static constexpr int BM = 16 * RT, BN = 16 * CT * NW, NT = 64 * NW;
    // DMA instructions of a slot, by kind: activation rows (16 chunks a row,
    // 64 an instruction), weight blocks (9 chunks a 144-byte block), the rows'
    // 16-element sums (two chunks a row), their scales (4 bytes a lane)
    static constexpr int CA = BM / 4, CW = (BN * 9 + 63) / 64, CS = (2 * BM + 63) / 64, CD = (BM + 63) / 64;
    // every wavefront issues FA + FW + FS + FD of them, then XR "extra" ones
    // from the remainders (the spare extras repeat the slot's last activation
    // load: same source, same bytes, same place)
    static constexpr int FA = CA / NW, FW = CW / NW, FS = CS / NW, FD = CD / NW;
    static constexpr int RA = CA % NW, RW = CW % NW, RS = CS % NW, RD = CD % NW;
    static constexpr int E = RA + RW + RS + RD, XR = (E + NW - 1) / NW;
    static constexpr int NI = FA + FW + FS + FD + XR;  // per wavefront and superblock
    static_assert(NI <= 63, "vmcnt range");
    static constexpr int LA = CA * 1024, LW = CW * 1024, LS = CS * 1024, LD = CD * 256;
    static constexpr int OW = LA, OS = LA + LW, OD = LA + LW + LS, LBUF = LA + LW + LS + LD;
};

// u16x2{v, v} of byte `sel` of w (a v_perm selector: bytes [b, 0, b, 0])
__device__ __forceinline__ uint32_t byte_pair(uint32_t w, uint32_t sel) { return __builtin_amdgcn_perm(0u, w, sel); }

__device__ __forceinline__ int bytes_times_p(uint32_t q, uint32_t f2) {
    const u16x2 p = __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, f2);
    return __builtin_bit_cast(int, p);
}

// KG > 1: KG groups of NW wavefronts share the tile, group g taking every
// KG-th superblock of the split (its own two LDS slots), and the groups' f32
// tiles are added through LDS in group order at the end -- a K split inside
// the workgroup, more wavefronts per tile without partials in memory or a
// reduce launch.  Every wavefront runs the same number of iterations (a group
// with no superblock left in the last one only waits at its barrier).
template <int RT, int CT, int NW, int KG = 1>
__global__ __launch_bounds__(64 * NW * KG) void mmq_q4k_wide_kernel(const uint8_t* __restrict__ W, ActView act,
                                                                    float* __restrict__ y, int M, int N, int K,
                                                                    int ldy, int mt, int nt, int ks, int out_mode) {
    using T = WideTile<RT, CT, NW>;
    constexpr int BM = T::BM, BN = T::BN;
    __shared__ __align__(16) uint8_t sB0[KG][T::LBUF], sB1[KG][T::LBUF];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = KG > 1 ? wave_all / NW : 0;  // (wave-uniform)
    const int wave = wave_all - grp * NW;        // within the group
    const int KB = K / QK_K;
    const uint32_t row_bytes = (uint32_t)KB * Q4K_BYTES;
    const int l16 = lane & 15, kb = lane >> 4;

    const int total = mt * nt, z = blockIdx.x / total, L = blockIdx.x - z * total;
    const int x = L & 7, slot = L >> 3, q8 = total >> 3, r8 = total & 7;
    const int tile = x * q8 + (x < r8 ? x : r8) + slot;  // XCD x's contiguous range of tiles
    const int mtile = tile % mt, ntile = tile / mt;
    const int m0 = mtile * BM, n0 = ntile * BN;
    // K split z of ks: superblocks [bs, be) into partial z (y then points at
    // the partials, ldy = N)
    const int per = (KB + ks - 1) / ks, bs = z * per, be = min(KB, bs + per);
    y += (size_t)z * M * ldy;

    // per-lane source byte offsets (superblock 0) of DMA instruction i of each
    // kind; rows past M read offset 0 and tail columns column N-1 (valid
    // addresses; those bytes are never used)
    auto a_src = [&](int i) {
        const int q = 64 * i + lane, r = q >> 4, m = m0 + r;
        return m < M ? (uint32_t)m * (uint32_t)K + 16u * (uint32_t)((q & 15) ^ (r & 15)) : 0u;
    };
    auto w_src = [&](int i) {
        const int q = 64 * i + lane;
        int n = n0 + q / 9;
        n = n < N ? n : N - 1;
        return (uint32_t)n * row_bytes + 16u * (uint32_t)(q % 9);
    };
    auto s_src = [&](int i) {
        const int q = 64 * i + lane, r = q >> 1, m = m0 + r;
        return r < BM && m < M ? 32u * (uint32_t)m * (uint32_t)KB + 16u * (uint32_t)(q & 1) : 0u;
    };
    auto d_src = [&](int i) {
        const int q = 64 * i + lane, m = m0 + q;
        return q < BM && m < M ? 4u * (uint32_t)m * (uint32_t)KB : 0u;
    };
    uint32_t asrc[T::FA > 0 ? T::FA : 1], wsrc[T::FW > 0 ? T::FW : 1], ssrc[T::FS > 0 ? T::FS : 1],
        dsrc[T::FD > 0 ? T::FD : 1], xsrc[T::XR > 0 ? T::XR : 1];
#pragma unroll
    for (int j = 0; j < T::FA; j++) asrc[j] = a_src(j * NW + wave);
#pragma unroll
    for (int j = 0; j < T::FW; j++) wsrc[j] = w_src(j * NW + wave);
#pragma unroll
    for (int j = 0; j < T::FS; j++) ssrc[j] = s_src(j * NW + wave);
#pragma unroll
    for (int j = 0; j < T::FD; j++) dsrc[j] = d_src(j * NW + wave);
    // extra x of this wavefront: remainder e = x NW + wave (wave-uniform kind)
#pragma unroll
    for (int x = 0; x < T::XR; x++) {
        const int e = x * NW + wave;
        if (e < T::RA) xsrc[x] = a_src(T::FA * NW + e);
        else if (e < T::RA + T::RW) xsrc[x] = w_src(T::FW * NW + e - T::RA);
        else if (e < T::RA + T::RW + T::RS) xsrc[x] = s_src(T::FS * NW + e - T::RA - T::RW);
        else if (e < T::E) xsrc[x] = d_src(T::FD * NW + e - T::RA - T::RW - T::RS);
        else xsrc[x] = a_src(T::CA - 1);
    }
    const uint8_t* qbase = reinterpret_cast<const uint8_t*>(act.qs);
    const uint8_t* sbase = reinterpret_cast<const uint8_t*>(act.bsh);
    const uint8_t* dbase = reinterpret_cast<const uint8_t*>(act.d);
    // (each DMA writes at the instruction's LDS base + lane * size)
    auto issue = [&](int b, uint32_t buf) __attribute__((always_inline)) {
        const uint32_t ub = (uint32_t)b;
#pragma unroll
        for (int j = 0; j < T::FA; j++) dma16_asm(qbase, asrc[j] + ub * QK_K, buf + (uint32_t)(1024 * (j * NW + wave)));
#pragma unroll
        for (int j = 0; j < T::FW; j++) dma16_asm(W, wsrc[j] + ub * Q4K_BYTES, buf + (uint32_t)(T::OW + 1024 * (j * NW + wave)));
#pragma unroll
        for (int j = 0; j < T::FS; j++) dma16_asm(sbase, ssrc[j] + ub * 32u, buf + (uint32_t)(T::OS + 1024 * (j * NW + wave)));
#pragma unroll
        for (int j = 0; j < T::FD; j++) dma4_asm(dbase, dsrc[j] + ub * 4u, buf + (uint32_t)(T::OD + 256 * (j * NW + wave)));
        // the extras: one branch per remainder slot, each with a compile-time
        // kind and LDS place (wave-uniform conditions)
        static_for<NW * T::XR>([&](auto ec) __attribute__((always_inline)) {
            constexpr int e = decltype(ec)::value, x = e / NW;
            if (wave != e % NW) return;
            if constexpr (e < T::RA) {
                dma16_asm(qbase, xsrc[x] + ub * QK_K, buf + (uint32_t)(1024 * (T::FA * NW + e)));
            } else if constexpr (e < T::RA + T::RW) {
                dma16_asm(W, xsrc[x] + ub * Q4K_BYTES, buf + (uint32_t)(T::OW + 1024 * (T::FW * NW + e - T::RA)));
            } else if constexpr (e < T::RA + T::RW + T::RS) {
                dma16_asm(sbase, xsrc[x] + ub * 32u, buf + (uint32_t)(T::OS + 1024 * (T::FS * NW + e - T::RA - T::RW)));
            } else if constexpr (e < T::E) {
                dma4_asm(dbase, xsrc[x] + ub * 4u, buf + (uint32_t)(T::OD + 256 * (T::FD * NW + e - T::RA - T::RW - T::RS)));
            } else {  // spare: the slot's last activation-row load again
                dma16_asm(qbase, xsrc[x] + ub * QK_K, buf + (uint32_t)(1024 * (T::CA - 1)));
            }
        });
    };
    // v_perm selectors of scale byte 2 (kb>>1) + (t>>1)
    const uint32_t sel0 = (uint32_t)(2 * (kb >> 1)) * 0x00010001u | 0x0c000c00u;
    const uint32_t sel1 = sel0 + 0x00010001u;
    // msum B operand: bytes 2 (kb&1), 2 (kb&1) + 1 of min word kb>>1
    const uint32_t msel = (uint32_t)(2 * (kb & 1)) * 0x01010101u + 0x01010000u;

    float facc[RT][CT][4];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) facc[r][c][i] = 0.0f;

    const int b1 = be;
    const uint32_t slot0 = lds_addr(sB0[grp]), slot1 = lds_addr(sB1[grp]);
    // this group's superblocks: bs + grp, bs + grp + KG, ... (< be)
    const int iters = (be - bs + KG - 1) / KG;
    if (bs + grp < be) issue(bs + grp, slot0);

    auto iter = [&](auto kr, int b) __attribute__((always_inline)) {
        constexpr int KR = decltype(kr)::value;
        const uint8_t* A = KR == 0 ? sB0[grp] : sB1[grp];
        const uint8_t* Wl = A + T::OW;
        const uint8_t* S = A + T::OS;
        const float* D = reinterpret_cast<const float*>(A + T::OD);
        // superblock b landed (the only loads in flight), in every wavefront
        __builtin_amdgcn_s_waitcnt(FRQ_VMCNT(0));
        compiler_fence();
        __builtin_amdgcn_s_barrier();
        compiler_fence();
        // the other slot was read in the previous iteration, which every
        // wavefront has left: the group's next superblock's DMA runs while b is
        // multiplied
        if (b + KG < b1) issue(b + KG, KR == 0 ? slot1 : slot0);
        if (KG > 1 && b >= b1) return;  // (this group has no superblock left)
        // column headers: d, dmin, the 6-bit scales split as 8 a + b, the mins
        float d[CT], dmin[CT];
        uint32_t aw[CT][2], bw[CT][2], mw[CT];
        uint4 hd[CT];
        const uint8_t* col[CT];
#pragma unroll
        for (int c = 0; c < CT; c++) {
            col[c] = Wl + (16 * (CT * wave + c) + l16) * Q4K_BYTES;
            hd[c] = *reinterpret_cast<const uint4*>(col[c]);
            const uint32_t sc0 = hd[c].y & 0x3f3f3f3fu;
            const uint32_t sc1 = (hd[c].w & 0x0f0f0f0fu) | (((hd[c].y >> 6) & 0x03030303u) << 4);
            const uint32_t mn0 = hd[c].z & 0x3f3f3f3fu;
            const uint32_t mn1 = ((hd[c].w >> 4) & 0x0f0f0f0fu) | (((hd[c].z >> 6) & 0x03030303u) << 4);
            d[c] = f16_to_f32(hd[c].x & 0xffffu);
            dmin[c] = f16_to_f32(hd[c].x >> 16);
            aw[c][0] = (sc0 >> 3) & 0x07070707u;
            aw[c][1] = (sc1 >> 3) & 0x07070707u;
            bw[c][0] = sc0 & 0x07070707u;
            bw[c][1] = sc1 & 0x07070707u;
            mw[c] = kb < 2 ? mn0 : mn1;
        }
        v4i acc[RT][CT][2];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int j = 8 * (t & 1) + 4 * (kb >> 1) + 2 * (t >> 1) + (kb & 1);  // activation chunk
            v4i afr[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) afr[r] = *reinterpret_cast<const v4i*>(A + (16 * r + l16) * QK_K + 16 * (j ^ l16));
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const uint4 rw = *reinterpret_cast<const uint4*>(col[c] + 16 + 64 * (t & 1) + 16 * kb);
                const uint32_t sh = t >= 2 ? 4u : 0u;
                const uint32_t qd[4] = {(rw.x >> sh) & 0x0f0f0f0fu, (rw.y >> sh) & 0x0f0f0f0fu,
                                        (rw.z >> sh) & 0x0f0f0f0fu, (rw.w >> sh) & 0x0f0f0f0fu};
                const uint32_t sel = t >= 2 ? sel1 : sel0;
                const uint32_t pa = byte_pair(aw[c][t & 1], sel), pb = byte_pair(bw[c][t & 1], sel);
                const v4i ba = v4i{bytes_times_p(qd[0], pa), bytes_times_p(qd[1], pa), bytes_times_p(qd[2], pa),
                                   bytes_times_p(qd[3], pa)};
                const v4i bb = v4i{bytes_times_p(qd[0], pb), bytes_times_p(qd[1], pb), bytes_times_p(qd[2], pb),
                                   bytes_times_p(qd[3], pb)};
                const v4i zero = v4i{0, 0, 0, 0};
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    acc[r][c][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], ba, t == 0 ? zero : acc[r][c][0], 0, 0, 0);
                    acc[r][c][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(afr[r], bb, t == 0 ? zero : acc[r][c][1], 0, 0, 0);
                }
            }
        }
        // msum on f16 MFMA, then the f32 step
        wh4 mb[CT];
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const uint32_t mm = __builtin_amdgcn_perm(0u, mw[c], msel);  // bytes m_lo, m_lo, m_hi, m_hi
            mb[c] = wh4{(_Float16)(mm & 0xffu), (_Float16)((mm >> 8) & 0xffu), (_Float16)((mm >> 16) & 0xffu),
                        (_Float16)(mm >> 24)};
        }
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const wh4 sa = *reinterpret_cast<const wh4*>(S + (16 * r + l16) * 32 + 8 * kb);  // b_{4kb..4kb+3}
            const float4 dx = *reinterpret_cast<const float4*>(D + 16 * r + 4 * kb);
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const wf4 ms = __builtin_amdgcn_mfma_f32_16x16x16f16(sa, mb[c], wf4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int isum = 8 * acc[r][c][0][i] + acc[r][c][1][i];
                    facc[r][c][i] = fmaf(dxv[i], fmaf(-dmin[c], ms[i], d[c] * (float)isum), facc[r][c][i]);
                }
            }
        }
    };
    for (int it = 0; it < iters; it += 2) {
        const int b = bs + grp + it * KG;
        iter(std::integral_constant<int, 0>{}, b);
        if (it + 1 < iters) iter(std::integral_constant<int, 1>{}, b + KG);
    }

    if constexpr (KG > 1) {
        // groups 1.. hand their tiles to group 0 through the (now free) slots
        constexpr int TILE = RT * CT * 4;
        static_assert((KG - 1) * NW * 64 * TILE * 4 <= KG * T::LBUF, "reduction fits the first slots");
        float* red = reinterpret_cast<float*>(&sB0[0][0]);
        __syncthreads();
        if (grp > 0) {
            float* dst = red + ((size_t)((grp - 1) * NW + wave) * TILE) * 64 + lane;
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int c = 0; c < CT; c++)
#pragma unroll
                    for (int i = 0; i < 4; i++) dst[64 * ((r * CT + c) * 4 + i)] = facc[r][c][i];
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int g = 1; g < KG; g++) {
            const float* src = red + ((size_t)((g - 1) * NW + wave) * TILE) * 64 + lane;
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int c = 0; c < CT; c++)
#pragma unroll
                    for (int i = 0; i < 4; i++) facc[r][c][i] += src[64 * ((r * CT + c) * 4 + i)];
        }
    }

#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int n = n0 + 16 * (CT * wave + c) + l16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * r + 4 * kb + i;
                if (m < M && n < N) store_out(y, (size_t)m * ldy + n, facc[r][c][i], out_mode);
            }
        }
}

// ---- Q6_K, wide tiles ----
// The same skeleton for Q6_K: NW wavefronts side by side in N share 16 RT
// activation rows, one 16-column tile each, so each weight block is turned
// into its byte planes once per workgroup; activation rows and scales come by
// DMA (the assembly issue above), two slots.  210-byte blocks are only 2-byte
// aligned, so the weights are staged through registers instead: the next
// superblock's 14 chunks per column (MmqQ6K's layout, 224 bytes a column) are
// loaded right after the barrier and stored to the other slot after the
// arithmetic.  Products, planes and the f32 step are MmqQ6K's.
template <int RT, int NW>
struct WideTile6 {
    using F = MmqQ6K;
    static constexpr int BM = 16 * RT, BN = 16 * NW, NT = 64 * NW;
    static constexpr int CA = BM / 4, CD = (BM + 63) / 64;
    static constexpr int FA = CA / NW, FD = CD / NW, RA = CA % NW, RD = CD % NW;
    static constexpr int E = RA + RD, XR = (E + NW - 1) / NW;
    static constexpr int W_CH = BN * F::CH, W_PT = (W_CH + NT - 1) / NT;
    static constexpr int LA = CA * 1024, LW = BN * F::STRIDE, LD = CD * 256;
    static constexpr int OW = LA, OD = LA + LW, LBUF = LA + LW + LD;
};

template <int RT, int NW>
__global__ __launch_bounds__(64 * NW) void mmq_q6k_wide_kernel(const uint8_t* __restrict__ W, ActView act,
                                                               float* __restrict__ y, int M, int N, int K, int ldy,
                                                               int mt, int nt, int out_mode) {
    using T = WideTile6<RT, NW>;
    using F = MmqQ6K;
    constexpr int BM = T::BM, BN = T::BN;
    __shared__ __align__(16) uint8_t sB0[T::LBUF], sB1[T::LBUF];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KB = K / QK_K;
    const uint32_t row_bytes = (uint32_t)KB * Q6K_BYTES;
    const int l16 = lane & 15, kb = lane >> 4;

    const int total = mt * nt, L = blockIdx.x;
    const int x = L & 7, slot = L >> 3, q8 = total >> 3, r8 = total & 7;
    const int tile = x * q8 + (x < r8 ? x : r8) + slot;  // XCD x's contiguous range of tiles
    const int mtile = tile % mt, ntile = tile / mt;
    const int m0 = mtile * BM, n0 = ntile * BN;

    auto a_src = [&](int i) {
        const int q = 64 * i + lane, r = q >> 4, m = m0 + r;
        return m < M ? (uint32_t)m * (uint32_t)K + 16u * (uint32_t)((q & 15) ^ (r & 15)) : 0u;
    };
    auto d_src = [&](int i) {
        const int q = 64 * i + lane, m = m0 + q;
        return q < BM && m < M ? 4u * (uint32_t)m * (uint32_t)KB : 0u;
    };
    uint32_t asrc[T::FA > 0 ? T::FA : 1], dsrc[T::FD > 0 ? T::FD : 1], xsrc[T::XR > 0 ? T::XR : 1];
#pragma unroll
    for (int j = 0; j < T::FA; j++) asrc[j] = a_src(j * NW + wave);
#pragma unroll
    for (int j = 0; j < T::FD; j++) dsrc[j] = d_src(j * NW + wave);
#pragma unroll
    for (int x = 0; x < T::XR; x++) {
        const int e = x * NW + wave;
        if (e < T::RA) xsrc[x] = a_src(T::FA * NW + e);
        else if (e < T::E) xsrc[x] = d_src(T::FD * NW + e - T::RA);
        else xsrc[x] = a_src(T::CA - 1);
    }
    // weight chunks of this thread: chunk idx = tid + i NT of the tile (column
    // idx / 14, MmqQ6K chunk idx % 14); tail columns re-read column N-1
    uint32_t wsrc[T::W_PT], wdst[T::W_PT];
#pragma unroll
    for (int i = 0; i < T::W_PT; i++) {
        const int idx = tid + i * T::NT;
        const int c = idx < T::W_CH ? idx / F::CH : 0, ch = idx % F::CH;
        int n = n0 + c;
        n = n < N ? n : N - 1;
        wsrc[i] = (uint32_t)n * row_bytes + F::src(ch);
        wdst[i] = (uint32_t)(T::OW + c * F::STRIDE + 16 * ch);
    }
    const uint8_t* qbase = reinterpret_cast<const uint8_t*>(act.qs);
    const uint8_t* dbase = reinterpret_cast<const uint8_t*>(act.d);
    auto issue = [&](int b, uint32_t buf) __attribute__((always_inline)) {
        const uint32_t ub = (uint32_t)b;
#pragma unroll
        for (int j = 0; j < T::FA; j++) dma16_asm(qbase, asrc[j] + ub * QK_K, buf + (uint32_t)(1024 * (j * NW + wave)));
#pragma unroll
        for (int j = 0; j < T::FD; j++) dma4_asm(dbase, dsrc[j] + ub * 4u, buf + (uint32_t)(T::OD + 256 * (j * NW + wave)));
        static_for<NW * T::XR>([&](auto ec) __attribute__((always_inline)) {
            constexpr int e = decltype(ec)::value, x = e / NW;
            if (wave != e % NW) return;
            if constexpr (e < T::RA) {
                dma16_asm(qbase, xsrc[x] + ub * QK_K, buf + (uint32_t)(1024 * (T::FA * NW + e)));
            } else if constexpr (e < T::E) {
                dma4_asm(dbase, xsrc[x] + ub * 4u, buf + (uint32_t)(T::OD + 256 * (T::FD * NW + e - T::RA)));
            } else {  // spare: the slot's last activation-row load again
                dma16_asm(qbase, xsrc[x] + ub * QK_K, buf + (uint32_t)(1024 * (T::CA - 1)));
            }
        });
    };
    uint4 wreg[T::W_PT];
    auto wload = [&](int b) __attribute__((always_inline)) {
        const uint32_t o = (uint32_t)b * Q6K_BYTES;
#pragma unroll
        for (int i = 0; i < T::W_PT; i++) {
            wreg[i] = uint4{0u, 0u, 0u, 0u};
            if (tid + i * T::NT < T::W_CH) wreg[i] = load16_u(W + (wsrc[i] + o));
        }
    };
    auto wstore = [&](uint8_t* buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < T::W_PT; i++)
            if (tid + i * T::NT < T::W_CH) *reinterpret_cast<uint4*>(buf + wdst[i]) = wreg[i];
    };

    float facc[RT][4];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) facc[r][i] = 0.0f;

    const int b1 = KB;
    const uint32_t slot0 = lds_addr(sB0), slot1 = lds_addr(sB1);
    issue(0, slot0);
    wload(0);
    wstore(sB0);

    auto iter = [&](auto kr, int b) __attribute__((always_inline)) {
        constexpr int KR = decltype(kr)::value;
        const uint8_t* A = KR == 0 ? sB0 : sB1;
        const uint8_t* Wl = A + T::OW;
        const float* D = reinterpret_cast<const float*>(A + T::OD);
        // superblock b landed (the DMA: vmcnt; this wavefront's weight stores:
        // lgkmcnt), in every wavefront
        __builtin_amdgcn_s_waitcnt(FRQ_VMCNT(0) & ~(0xF << 8));
        compiler_fence();
        __builtin_amdgcn_s_barrier();
        compiler_fence();
        // the other slot was read in iteration b-1: b+1's loads run while b is multiplied
        const bool more = b + 1 < b1;
        if (more) {
            issue(b + 1, KR == 0 ? slot1 : slot0);
            wload(b + 1);
        }
        const uint8_t* col = Wl + (16 * wave + l16) * F::STRIDE;
        typename F::Hdr hdr;
        F::header(col, hdr);
        v4i acc[RT][1][F::NACC];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            v4i afr[RT];
#pragma unroll
            for (int r = 0; r < RT; r++)
                afr[r] = *reinterpret_cast<const v4i*>(A + (16 * r + l16) * QK_K + 16 * ((4 * t + kb) ^ l16));
            F::template step<RT, 1>(t, kb, 0, col, hdr, afr, acc);
        }
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const float4 dx = *reinterpret_cast<const float4*>(D + 16 * r + 4 * kb);
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int i = 0; i < 4; i++) facc[r][i] = fmaf(dxv[i], F::finish(acc[r][0], i, hdr), facc[r][i]);
        }
        if (more) wstore(KR == 0 ? sB1 : sB0);
    };
    for (int b = 0; b < b1; b += 2) {
        iter(std::integral_constant<int, 0>{}, b);
        if (b + 1 < b1) iter(std::integral_constant<int, 1>{}, b + 1);
    }
    __builtin_amdgcn_s_waitcnt(FRQ_VMCNT(0));

    const int n = n0 + 16 * wave + l16;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + 16 * r + 4 * kb + i;
            if (m < M && n < N) store_out(y, (size_t)m * ldy + n, facc[r][i], out_mode);
        }
}

template <int RT, int NW>
hipError_t launch_wide6(const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy, hipStream_t s,
                        int out_mode) {
    using T = WideTile6<RT, NW>;
    const int mt = (M + T::BM - 1) / T::BM, nt = (N + T::BN - 1) / T::BN;
    hipLaunchKernelGGL((mmq_q6k_wide_kernel<RT, NW>), dim3(mt * nt), dim3(T::NT), 0, s, w, act, y, M, N, K, ldy, mt,
                       nt, out_mode);
    return hipGetLastError();
}


// y[m][n] = sum over splits z (in order) of part[z][m][n]
__global__ void mmq_reduce_kernel(const float* __restrict__ part, float* __restrict__ y, int M, int N, int ldy,
                                  int nsplit, int out_mode) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * N) return;
    float s = part[i];
    for (int z = 1; z < nsplit; z++) s += part[(size_t)z * M * N + i];
    const size_t o = (i / N) * ldy + i % N;
    store_out(y, o, s, out_mode);
}

// The wide Q4_K kernel, over ks K splits (ks > 1: into part[ks][M][N], then
// mmq_reduce_kernel adds them in split order into y), KG wavefront groups per
// tile.
template <int RT, int CT, int NW, int KG = 1>
hipError_t launch_wide(const uint8_t* w, ActView act, float* y, int M, int N, int K, int ldy, hipStream_t s,
                       int out_mode, int ks = 1, float* part = nullptr) {
    using T = WideTile<RT, CT, NW>;
    const int mt = (M + T::BM - 1) / T::BM, nt = (N + T::BN - 1) / T::BN;
    if (ks > 1 && !part) return hipErrorInvalidValue;
    if (ks > 1)
        hipLaunchKernelGGL((mmq_q4k_wide_kernel<RT, CT, NW, KG>), dim3(mt * nt * ks), dim3(T::NT * KG), 0, s, w, act,
                           part, M, N, K, N, mt, nt, ks, 0);
    else
        hipLaunchKernelGGL((mmq_q4k_wide_kernel<RT, CT, NW, KG>), dim3(mt * nt), dim3(T::NT * KG), 0, s, w, act, y, M,
                           N, K, ldy, mt, nt, 1, out_mode);
    if (ks > 1) {
        const size_t total = (size_t)M * N;
        hipLaunchKernelGGL(mmq_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, y, M, N,
                           ldy, ks, out_mode);
    }
    return hipGetLastError();
}

// Resident workgroups per CU of one kernel instantiation at `Threads` threads
// per workgroup.  The template parameter is the kernel itself, so every
// instantiation has its own cache (kernels of one signature do not share it):
// a plan is a function of its call alone, never of which kernels were planned
// before in the process.  The first query initialises the static (thread-safe).
template <auto Kern, int Threads>
int kernel_occupancy() {
    static const int occ = [] {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, Kern, Threads, 0) != hipSuccess || o < 1) o = 1;
        return o;
    }();
    return occ;
}

// K splits for a grid of `tiles` workgroups: split when the tiles leave
// resident workgroup slots empty, as far as one round of the grid still fits
// them (a partial second round costs more than the split saves), keeping >= 2
// superblocks per split and at most 16 splits.
int mmq_ksplit(int tiles, int occ, int num_cus, int KB) {
    const int cap = occ * num_cus;
    if (tiles >= cap) return 1;
    int ks = cap / tiles;
    const int kmax = KB / 2 > 1 ? KB / 2 : 1;
    if (ks > kmax) ks = kmax;
    return ks > 16 ? 16 : ks;
}

template <class F, int RT, int CT, int WM, int WN, bool DMA>
void plan_cfg(int M, int N, int K, int num_cus, MmqPlan& p) {
    constexpr int NT = 64 * WM * WN, BM = 16 * RT * WM, BN = 16 * CT * WN;
    const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    int occ;
    if constexpr (DMA) occ = kernel_occupancy<mmq_dma_kernel<F, RT, CT, WM, WN, false>, NT>();
    else occ = kernel_occupancy<mmq_kernel<F, RT, CT, WM, WN, false>, NT>();
    p.ks = mmq_ksplit(mt * nt, occ, num_cus, K / QK_K);
    p.part_elems = p.ks > 1 ? (size_t)p.ks * M * N : 0;
}

template <class F, int RT, int CT, int WM, int WN, bool DMA>
hipError_t launch_cfg(const MmqPlan& p, const uint8_t* w, ActView act, float* y, float* part, int M, int N, int K,
                      int ldy, hipStream_t s, int out_mode) {
    constexpr int NT = 64 * WM * WN, BM = 16 * RT * WM, BN = 16 * CT * WN;
    const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    const int ks = p.ks;
    if (ks > 1 && !part) return hipErrorInvalidValue;
    float* out = ks > 1 ? part : y;
    if constexpr (DMA)
        hipLaunchKernelGGL((mmq_dma_kernel<F, RT, CT, WM, WN, false>), dim3(mt * nt * ks), dim3(NT), 0, s, w, act, out,
                           M, N, K, ldy, mt, nt, ks, out_mode, MmqGroup{});
    else
        hipLaunchKernelGGL((mmq_kernel<F, RT, CT, WM, WN, false>), dim3(mt * nt * ks), dim3(NT), 0, s, w, act, out, M,
                           N, K, ldy, mt, nt, ks, out_mode, MmqGroup{});
    if (ks > 1) {
        const size_t total = (size_t)M * N;
        hipLaunchKernelGGL(mmq_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, y, M, N,
                           ldy, ks, out_mode);
    }
    return hipGetLastError();
}

template <class F, int RT, int CT, int WM, int WN>
hipError_t launch_grouped_cfg(const uint8_t* w, ActView act, float* y, int max_tiles, int N, int K, int ldy,
                              const MmqGroup& g, hipStream_t s) {
    using T = MmqTile<F, RT, CT, WM, WN>;
    dim3 grid(max_tiles, (N + T::BN - 1) / T::BN, 1);
    hipLaunchKernelGGL((mmq_kernel<F, RT, CT, WM, WN, true>), grid, dim3(T::NT), 0, s, w, act, y, 0, N, K, ldy, 0, 0,
                       1, 0, g);
    return hipGetLastError();
}

template <class F>
hipError_t launch_grouped_fmt(const uint8_t* w, ActView act, float* y, int bm, int max_tiles, int N, int K, int ldy,
                              const MmqGroup& g, hipStream_t s) {
    // 32 x 128 (eight wavefronts side by side: each activation tile feeds twice
    // the columns; MoE T = 512 layer 212 -> 198 us, bit-identical) where the
    // W | W2 split allows it, else 32 x 64
    if (bm == 32 && (!g.w2 || g.n_split % 128 == 0))
        return launch_grouped_cfg<F, 2, 1, 1, 8>(w, act, y, max_tiles, N, K, ldy, g, s);
    if (bm == 32) return launch_grouped_cfg<F, 2, 1, 1, 4>(w, act, y, max_tiles, N, K, ldy, g, s);  // 32 x 64
    if (bm == 16) return launch_grouped_cfg<F, 1, 1, 1, 4>(w, act, y, max_tiles, N, K, ldy, g, s);  // 16 x 64
    return hipErrorInvalidValue;
}

// Kernel instantiations, by MmqPlan::kind.
enum MmqKind {
    MMQ_Q4K_32 = 0,   // register-staged 32 x 64
    MMQ_Q4K_64,       // register-staged 64 x 64
    MMQ_Q4K_128,      // register-staged 128 x 64, 8 waves
    MMQ_Q4K_DMA_64,   // LDS-DMA 64 x 64 (16-byte aligned blocks)
    MMQ_Q4K_DMA_128,  // LDS-DMA 128 x 64
    MMQ_Q6K_32,
    MMQ_Q6K_64,
    MMQ_Q6K_128,
    MMQ_Q4K_WIDE,      // 64 x 128, eight wavefronts side by side in N (16-byte aligned Q4_K blocks)
    MMQ_Q6K_WIDE,      // 64 x 128, the same for Q6_K
    MMQ_Q4K_WIDE32,    // 32 x 64, the wide-tile kernel with four wavefronts (grids of few 64 x 128 tiles)
    MMQ_Q4K_WIDE_KG2,    // 64 x 128, two groups of eight wavefronts splitting K inside the workgroup
    MMQ_Q4K_WIDE32_KG2,  // 32 x 64, two groups of four wavefronts
    MMQ_Q4K_WIDE16_KG2,  // 16 x 64, two groups of four wavefronts
    MMQ_Q6K_WIDE16,      // 16 x 64, the Q6_K wide-tile kernel with four wavefronts
    MMQ_Q6K_WIDE32,      // 32 x 64, the same
};

#define FRQ_MMQ_KINDS(X)                          \
    X(MMQ_Q4K_32, MmqQ4K, 2, 1, 1, 4, false)      \
    X(MMQ_Q4K_64, MmqQ4K, 2, 2, 2, 2, false)      \
    X(MMQ_Q4K_128, MmqQ4K, 4, 1, 2, 4, false)     \
    X(MMQ_Q4K_DMA_64, MmqQ4K, 2, 2, 2, 2, true)   \
    X(MMQ_Q4K_DMA_128, MmqQ4K, 4, 1, 2, 4, true)  \
    X(MMQ_Q6K_32, MmqQ6K, 2, 1, 1, 4, false)      \
    X(MMQ_Q6K_64, MmqQ6K, 2, 2, 2, 2, false)      \
    X(MMQ_Q6K_128, MmqQ6K, 4, 1, 2, 4, false)

}  // namespace

bool mmq_supported(int dtype) { return dtype == GGML_Q4K || dtype == GGML_Q6K; }


MmqPlan mmq_plan(int dtype, const void* w, int M, int N, int K, int num_cus, size_t max_part_elems) {
    MmqPlan p{};
    // 144-byte Q4_K blocks at a 16-byte aligned base allow the LDS DMA staging
    // (16-byte global_load_lds); it wins from M = 64 on (M = 512: 4-7%), the
    // register-staged kernel below that
    const bool dma = dtype == GGML_Q4K && ((uintptr_t)w & 15u) == 0;
    const int base = dtype == GGML_Q4K ? MMQ_Q4K_32 : MMQ_Q6K_32;
    p.kind = M >= 128 ? base + 2 : M >= 64 ? base + 1 : base;
    if (dma && M >= 64) p.kind = M >= 128 ? MMQ_Q4K_DMA_128 : MMQ_Q4K_DMA_64;
    // Q6_K: 32-row tiles up to 64 rows, 128-row tiles above (a 96-row call in
    // one partly empty 128-row tile: 4096x4096 22.6 -> 19.3 us, 4096x11008
    // 54.1 -> 36.5, 11008x4096 41.7 -> 33.0, 4096x32000 109.3 -> 72.8 against
    // two 64-row tiles)
    if (dtype == GGML_Q6K) p.kind = M > 64 ? MMQ_Q6K_128 : MMQ_Q6K_32;
    switch (p.kind) {
#define FRQ_PLAN(kind, F, RT, CT, WM, WN, DMA) \
    case kind: plan_cfg<F, RT, CT, WM, WN, DMA>(M, N, K, num_cus, p); break;
        FRQ_MMQ_KINDS(FRQ_PLAN)
#undef FRQ_PLAN
        default: break;
    }
    // (Q6_K: at most four splits; six measured slower, 4096x4096 M = 33 15.9
    // against 15.3 us, 11008x4096 28.2 against 28.1)
    if (dtype == GGML_Q6K && p.ks > 4) p.ks = 4;
    while (p.ks > 1 && (size_t)p.ks * M * N > max_part_elems) p.ks--;
    // Q4_K at a 16-byte aligned base from 33 rows: the wide-tile kernel (two
    // MFMAs per product instead of three, the DMA ring out of the compiler's
    // sight; 19-25% faster than the plane kernels at M = 512 on the 7B shapes),
    // in one of two tiles by how its 64 x 128 tiles fill the chip (t8 of them
    // against C CUs; two resident per CU):
    // * long rows (K >= 8192) from 128 rows while t8 < 0.8 C: 64 x 128 with a
    //   K split of up to four, as many as one round of resident workgroups
    //   holds (11008x4096 M = 128 25.3 against 26.5 us with eight splits);
    // * 0.8 C <= t8 <= C (long rows from 128 rows: up to 1.25 C): 64 x 128
    //   with two wavefront groups splitting K inside the workgroup (11008x4096
    //   M = 512 57.4 against 61.5 us with two splits in memory, 4096x4096 M =
    //   512 25.1 against 26.4 us with one group, 4096x32000 M = 64 equal);
    // * t8 >= 1.25 C: 64 x 128, no K split (4096x32000 at M = 64 29.8 against
    //   35.0 us with two splits and 37.8 us in 32 x 64 tiles);
    // * otherwise, grids well short of one workgroup per CU or just past it
    //   (two on a few CUs), 32 x 64 tiles of four wavefronts, four resident
    //   per CU, K split while they are short of one round (long rows: four
    //   splits below 3 C tiles); at most one per CU with short rows, two
    //   wavefront groups per tile (4096x4096 M = 128 15.2 -> 12.8 us, M = 64
    //   12.5 -> 11.7 with two splits).  Against the previous plan (the plane kernels
    //   below 128 rows, 64 x 128 above): 4096x4096 M = 64 14.6 -> 12.3 us,
    //   M = 128 19.4 -> 15.2, M = 256 25.3 -> 19.0, M = 384 26.9 -> 25.5;
    //   4096x11008 M = 64 25.2 -> 20.1, M = 128 27.5 -> 26.1, M = 160 38.4 ->
    //   31.4; 11008x4096 M = 64 22.3 -> 19.4 (graph replays, weights rotated
    //   over 1.2 GB, split-K reduce included).
    // 16-32 rows (tiled on >= 8192 columns, and on rows of >= 8192 elements
    // from 24 rows): the 32 x 64 tiles, or 16 x 64 at 16 rows -- long rows
    // with a K split of up to four (11008x4096 M = 24 17.1 -> 15.5 us, M = 32
    // 19.9 -> 15.6 against the skinny kernel), two wavefront groups while the
    // tiles fit one per CU (4096x11008 M = 16 15.4 -> 12.0 us, M = 24 16.2 ->
    // 13.5, M = 32 16.6 -> 14.1; a K split in memory measured slower there),
    // one group above (4096x32000 M = 24 26.8 -> 21.6, M = 32 27.6 -> 23.4;
    // 16 x 64 tiles with two groups at M = 16 27.1 -> 18.6 us) -- against the
    // 32 x 64 plane kernel (graph replays, weights rotated over 1.2 GB, split-K
    // reduce included).  The 16 x 64 tiles also take 3-15 rows of >= 8192
    // columns (the caller's row rule): 4096x32000 M = 4 16.3 us, M = 8 16.8,
    // M = 12 17.4 against 27 us for the 32 x 64 plane kernel.
    if (dma && M >= 2) {
        using T8 = WideTile<4, 1, 8>;
        using T4 = WideTile<2, 1, 4>;
        const int KB = K / QK_K, C = num_cus;
        const bool long_rows = K >= 32 * QK_K;
        const int t8 = ((M + T8::BM - 1) / T8::BM) * ((N + T8::BN - 1) / T8::BN);
        const int t4 = ((M + T4::BM - 1) / T4::BM) * ((N + T4::BN - 1) / T4::BN);
        auto clamp_ks = [&](int ks) {
            if (ks > 4) ks = 4;
            if (ks > KB / 2) ks = KB / 2;
            return ks > 1 ? ks : 1;
        };
        if (M <= 32) {
            p.ks = 1;
            if (long_rows) {
                p.kind = MMQ_Q4K_WIDE32;
                p.ks = clamp_ks((3 * C + t4 - 1) / t4);
            } else if (M <= 16) {
                p.kind = MMQ_Q4K_WIDE16_KG2;
            } else {
                p.kind = t4 <= C ? MMQ_Q4K_WIDE32_KG2 : MMQ_Q4K_WIDE32;
            }
        } else if (long_rows && M >= 128 && t8 < 4 * C / 5) {
            const int occ = kernel_occupancy<mmq_q4k_wide_kernel<4, 1, 8>, T8::NT>();
            p.kind = MMQ_Q4K_WIDE;
            p.ks = clamp_ks(occ * C / t8);
        } else if ((t8 >= 4 * C / 5 && t8 <= C) || (long_rows && M >= 128 && t8 < 5 * C / 4)) {
            p.kind = MMQ_Q4K_WIDE_KG2;
            p.ks = 1;
        } else if (t8 >= 5 * C / 4) {
            p.kind = MMQ_Q4K_WIDE;
            p.ks = 1;
        } else {
            p.kind = MMQ_Q4K_WIDE32;
            if (long_rows) {
                p.ks = clamp_ks((3 * C + t4 - 1) / t4);
            } else if (t4 <= C) {
                p.kind = MMQ_Q4K_WIDE32_KG2;
                p.ks = t4 >= 3 * C / 4 ? 1 : clamp_ks((C + t4 - 1) / t4);
            } else {
                p.ks = 1;
            }
        }
        while (p.ks > 1 && (size_t)p.ks * M * N > max_part_elems) p.ks--;
    }
    // Q6_K from 128 rows without a K split, or from 33 rows when its 64 x 128
    // tiles fill 0.8-1 workgroups per CU (4096x32000 at M = 33-64: 64 -> 40 us
    // against the 32-row plane tiles): the wide-tile kernel
    // Q6_K at 5-32 rows of >= 24576 columns and rows of < 8192 elements (the
    // caller's row rule): 16 x 64 or 32 x 64 wide tiles of four wavefronts, no
    // K split -- 4096x32000 M = 8 35.9 -> 30.8 us, M = 16 35.8 -> 30.5, M = 32
    // 35.9 -> 34.5 against the 32 x 64 plane kernel, 40.0 / 44.2 / 67.2 on
    // the skinny kernel (graph replays, weights rotated over 1.2 GB)
    if (dtype == GGML_Q6K && M <= 32 && N >= 24576 && K < 32 * QK_K) {
        p.kind = M <= 16 ? MMQ_Q6K_WIDE16 : MMQ_Q6K_WIDE32;
        p.ks = 1;
    }
    if (dtype == GGML_Q6K && M >= 33) {
        using T6 = WideTile6<4, 8>;
        const int t8 = ((M + T6::BM - 1) / T6::BM) * ((N + T6::BN - 1) / T6::BN);
        if ((M >= 128 && p.ks == 1) || (t8 >= 4 * num_cus / 5 && t8 <= num_cus)) {
            p.kind = MMQ_Q6K_WIDE;
            p.ks = 1;
        }
    }
    p.part_elems = p.ks > 1 ? (size_t)p.ks * M * N : 0;
    return p;
}

hipError_t launch_mmq(const MmqPlan& plan, int dtype, const uint8_t* w, ActView act, float* y, float* part, int M,
                      int N, int K, int ldy, hipStream_t s, int out_mode) {
    if (!mmq_supported(dtype)) return hipErrorInvalidValue;
    switch (plan.kind) {
#define FRQ_LAUNCH(kind, F, RT, CT, WM, WN, DMA) \
    case kind: return launch_cfg<F, RT, CT, WM, WN, DMA>(plan, w, act, y, part, M, N, K, ldy, s, out_mode);
        FRQ_MMQ_KINDS(FRQ_LAUNCH)
#undef FRQ_LAUNCH
        case MMQ_Q4K_WIDE: return launch_wide<4, 1, 8>(w, act, y, M, N, K, ldy, s, out_mode, plan.ks, part);
        case MMQ_Q6K_WIDE: return launch_wide6<4, 8>(w, act, y, M, N, K, ldy, s, out_mode);
        case MMQ_Q4K_WIDE32: return launch_wide<2, 1, 4>(w, act, y, M, N, K, ldy, s, out_mode, plan.ks, part);
        case MMQ_Q4K_WIDE_KG2: return launch_wide<4, 1, 8, 2>(w, act, y, M, N, K, ldy, s, out_mode, plan.ks, part);
        case MMQ_Q4K_WIDE32_KG2:
            return launch_wide<2, 1, 4, 2>(w, act, y, M, N, K, ldy, s, out_mode, plan.ks, part);
        case MMQ_Q4K_WIDE16_KG2:
            return launch_wide<1, 1, 4, 2>(w, act, y, M, N, K, ldy, s, out_mode, plan.ks, part);
        case MMQ_Q6K_WIDE16: return launch_wide6<1, 4>(w, act, y, M, N, K, ldy, s, out_mode);
        case MMQ_Q6K_WIDE32: return launch_wide6<2, 4>(w, act, y, M, N, K, ldy, s, out_mode);
        default: return hipErrorInvalidValue;
    }
}

int mmq_group_rows(int rows_per_expert) { return rows_per_expert >= 24 ? 32 : 16; }

hipError_t launch_mmq_grouped(int dtype, const uint8_t* w, ActView act, float* y, int bm, int max_tiles, int N, int K,
                              int ldy, const MmqGroup& g, hipStream_t s) {
    if (!mmq_supported(dtype) || max_tiles <= 0) return max_tiles == 0 ? hipSuccess : hipErrorInvalidValue;
    if (g.w2 && g.n_split % 64) return hipErrorInvalidValue;  // a column tile must not straddle W | W2
    // (the register-staged kernel: the LDS DMA one measured 4-10% slower on the
    // MoE layer's short K loops)
    if (dtype == GGML_Q4K) return launch_grouped_fmt<MmqQ4K>(w, act, y, bm, max_tiles, N, K, ldy, g, s);
    return launch_grouped_fmt<MmqQ6K>(w, act, y, bm, max_tiles, N, K, ldy, g, s);
}

}  // namespace frq
