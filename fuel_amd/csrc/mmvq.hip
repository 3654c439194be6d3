// Quantized mat-vec for decode-sized M: fuel's matmul<T> (k_quants.rs:2284-2331)
// for T = BlockQ4K / BlockQ6K / BlockQ8_0, including the activation quantize
// step, in one kernel.
//
// Each workgroup first quantizes its activation row (f32 -> Q8K / Q8_0, the
// bit-exact routine of q8.hpp) into LDS: the activation loads are issued
// first, then the first weight row's, so the quantize step overlaps the HBM
// latency of the weights.  Then every wavefront walks weight rows with a grid
// stride: LPB lanes per block, 64/LPB blocks of one row per step, the next
// row's 128-bit weight loads in flight (a two-row register ring, no copies)
// while the current row is reduced.  Activation slices are read from LDS,
// scales/mins are unpacked in registers, the integer block sums use
// v_dot4_i32_i8 and each row ends in a DPP wave64 reduction.
//
// The only rounding after the exact integer stage is the f32 combination
// y += d_w*d_x*isum - dmin_w*d_x*msum.
#include "attn.hpp"
#include "common.hpp"
#include "formats.hpp"
#include "kernels.hpp"
#include "q8.hpp"
#include "qmv.hpp"
#include "route.hpp"

namespace frq {

// QMV_HALF: f16 activations in (x holds halves), f16 outputs (y holds
// halves, f16::from_f32 = round to nearest even of the f32 row sum).
// QMV_ATTN: x holds decode-attention split partials; the activation row is
// their merge (attn_merge_step), residual add as QMV_FUSED.
// QMV_GLU: activation as QMV_FUSED (RMS norm optional); output r is
// silu(gate_r . a) * (up_r . a) with gate rows in W and up rows in ix.w2.
// QMV_FUSED_NOX: QMV_FUSED without x2 and RMS norm (its own instantiation:
// with the run-time choice of activation loader compiled out, nothing merges
// registers at a join, so the first weight rows are requested before the
// activation row has arrived).
// QMV_INDEXED_ROUTE: QMV_INDEXED with the expert of each launch row picked in
// the workgroup from the token's router logits (route.hpp).
// QMV_GLU_RMS: QMV_GLU with the RMS norm and no second input, fixed at
// compile time (the decode step's gate|up launch).  With the choices made at
// run time the compiler's waits after each join assume the loads of either
// side (its norm waited for the first weight rows; gate|up 4096x11008 12.22
// -> 11.85 us with this instantiation and the store-free ring below).  The
// same for QMV_FUSED measured no faster (the q|k + v pair and the logits).
// The 16-lane row quantize (act16_*) from this many rounds of the 64-lane one.
#ifndef QMV_QUAD_MIN_ROUNDS
#define QMV_QUAD_MIN_ROUNDS 3
#endif

enum QmvMode {
    QMV_PLAIN = 0,
    QMV_INDEXED = 1,
    QMV_FUSED = 2,
    QMV_HALF = 3,
    QMV_ATTN = 4,
    QMV_GLU = 5,
    QMV_FUSED_NOX = 6,
    QMV_INDEXED_ROUTE = 7,
    QMV_GLU_RMS = 9
};

// Activation stage of QMV_ATTN: lane `lane`'s four elements of chunk
// w + NW*i are elements d..d+3 of head hd (HD = ATTN_HEAD_DIM per head; the
// 32 lanes of each half-wavefront share one head).  The partials of its (at
// most ATTN_MERGE_CHUNK = 8) splits are loaded with the other activation
// loads (attn_row_load) and merged once the first weight rows are requested
// (attn_row_merge).  Each lane loads the four output partials of every split
// but only one split's (max, sum) -- split lane & 7 of its head -- and turns
// it into that split's factor e^(m_s - M); the 8-lane groups share the
// factors and sums through swizzles.  The arithmetic per output element is
// attn_merge_step's, in the same order, so the outputs are the same bits as
// attn_combine_kernel's (against every lane loading all eight (max, sum)
// pairs and taking all eight exponentials: 4096x4096 o-projection 6.95 ->
// 6.2 us).
template <int MAXQ>
struct AttnRowPre {
    float4 o[MAXQ][ATTN_MERGE_CHUNK];
    float2 ml[MAXQ];  // (max, sum) of split lane & 7 (clamped to the last split)
};

template <int NW, int MAXQ>
__device__ __forceinline__ void attn_row_load(const float* __restrict__ part, int nsplit, int K, int w, int lane,
                                              AttnRowPre<MAXQ>& p) {
    const int nchunks = K / QK_K;
    const int sl = (lane & 7) < nsplit ? (lane & 7) : nsplit - 1;
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {
        const int e = act_elem(w + NW * i, nchunks, K, lane);
        const float* ph = part + (size_t)(e / ATTN_HEAD_DIM) * nsplit * ATTN_PSTRIDE + e % ATTN_HEAD_DIM;
        const float* pm = part + (size_t)(e / ATTN_HEAD_DIM) * nsplit * ATTN_PSTRIDE + ATTN_HEAD_DIM;
#pragma unroll
        for (int c = 0; c < ATTN_MERGE_CHUNK; c++) {
            const size_t so = (size_t)(c < nsplit ? c : nsplit - 1) * ATTN_PSTRIDE;
            p.o[i][c] = *reinterpret_cast<const float4*>(ph + so);
        }
        p.ml[i] = *reinterpret_cast<const float2*>(pm + (size_t)sl * ATTN_PSTRIDE);
    }
}

// Lane (lane & ~7) + C's v within each 8-lane group (ds_swizzle bit mode:
// and-mask 0x18, or-mask C, within 32-lane halves).
template <int C>
__device__ __forceinline__ float grp8_take(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (C << 5)));
}

template <int NW, int MAXQ>
__device__ __forceinline__ void attn_row_merge(const AttnRowPre<MAXQ>& p, int nsplit, bool pos_ok,
                                               ActRowPre<MAXQ>& out) {
    static_assert(ATTN_MERGE_CHUNK == 8, "one split per lane of an 8-lane group");
    const int lane = (int)(threadIdx.x & 63);
    const bool valid = (lane & 7) < nsplit;  // (a repeated split: factor 0, as attn_merge_step drops it)
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {
        // M = max over the valid splits (fmaxf: any order gives the same value)
        const float ms = valid ? p.ml[i].x : -__builtin_inff();
        float M = ms;
#define FRQ_DPP_MAX(ctrl) \
    M = fmaxf(M, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, M), ctrl, 0xF, 0xF, false)))
        FRQ_DPP_MAX(0xB1);   // quad_perm [1,0,3,2]
        FRQ_DPP_MAX(0x4E);   // quad_perm [2,3,0,1]
        FRQ_DPP_MAX(0x141);  // row_half_mirror: each 8-lane group holds its max
#undef FRQ_DPP_MAX
        // split 0 is never empty, so M is finite: an empty range's factor is 0
        const float fs = valid ? expf(ms - M) : 0.0f;
        const float ls = p.ml[i].y;
        const float f[8] = {grp8_take<0>(fs), grp8_take<1>(fs), grp8_take<2>(fs), grp8_take<3>(fs),
                            grp8_take<4>(fs), grp8_take<5>(fs), grp8_take<6>(fs), grp8_take<7>(fs)};
        const float l[8] = {grp8_take<0>(ls), grp8_take<1>(ls), grp8_take<2>(ls), grp8_take<3>(ls),
                            grp8_take<4>(ls), grp8_take<5>(ls), grp8_take<6>(ls), grp8_take<7>(ls)};
        float L = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < ATTN_MERGE_CHUNK; c++) {
            L = fmaf(l[c], f[c], L);
            O[0] = fmaf(p.o[i][c].x, f[c], O[0]);
            O[1] = fmaf(p.o[i][c].y, f[c], O[1]);
            O[2] = fmaf(p.o[i][c].z, f[c], O[2]);
            O[3] = fmaf(p.o[i][c].w, f[c], O[3]);
        }
        const float nan = __builtin_nanf("");
        out.v[i] = pos_ok ? make_float4(O[0] / L, O[1] / L, O[2] / L, O[3] / L) : make_float4(nan, nan, nan, nan);
    }
}

// Sum over the workgroup of one float per wavefront (valid in lane 63 of each
// wavefront), broadcast to every thread.
template <int NW>
__device__ __forceinline__ float block_sum_waves(float v, float* s_red, int w, int lane) {
    if (lane == 63) s_red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; i++) t += s_red[i];
    return t;
}

// The mat-vec of one workgroup: block bx of gxn walking the rows of W.
// RPW > 1 (rows of at most 16/RPW superblocks, SPL == 1): a wavefront step
// covers RPW consecutive rows, 16/RPW block slots each, instead of one row
// with most slots past its end; `row` then counts groups of RPW rows.
template <class F, int SPL, int WG, int MODE, int RPW = 1, int MR = 1>
__device__ __forceinline__ void qmv_body(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                         float* __restrict__ y, int N, int K, int ldy, const QmvOpts& ix, int bx,
                                         int gxn, uint8_t* smem, float* s_red, float* s_rt = nullptr,
                                         int* s_pick = nullptr) {
    constexpr int NW = WG / 64;
    static_assert(MR == 1 || (MODE == QMV_PLAIN && RPW == 1), "several rows per workgroup: the plain mode");
    const int m = blockIdx.y * MR;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int gi = lane / F::LPB, c = lane % F::LPB;
    const int KB = K / F::ELEMS;
    const size_t row_bytes = (size_t)KB * F::BYTES;
    const ActLds lay = act_lds_layout(F::ACT, K, F::QSTRIDE);
    int8_t* s_qs = reinterpret_cast<int8_t*>(smem);
    float* s_d = reinterpret_cast<float*>(smem + lay.off_d);
    int16_t* s_bs = reinterpret_cast<int16_t*>(smem + lay.off_bs);
    const int nw = gxn * NW;
    int row = bx * NW + w;
    const float* xr = x + (size_t)m * K;
    const uint8_t* W2 = W;
    int n_split = N;
    const float* xr2 = nullptr;
    if constexpr (MODE == QMV_INDEXED) {  // MoE: gathered activation row, per-row expert, optional second matrix
        const int sel = ix.w_sel[m];
        if ((unsigned)sel >= (unsigned)ix.n_experts) {  // uniform over the workgroup
            for (int r = bx * WG + threadIdx.x; r < N; r += gxn * WG) y[(size_t)m * ldy + r] = __builtin_nanf("");
            return;
        }
        const size_t xo = (size_t)(ix.x_row ? ix.x_row[m] : m / ix.x_div) * ix.ldx;
        xr = x + xo;
        if (ix.x2) xr2 = ix.x2 + xo;
        const size_t eoff = (size_t)sel * ix.expert_bytes;
        W += eoff;
        if (ix.w2) {
            W2 = ix.w2 + eoff;
            n_split = ix.n_split;
        }
    }
    float lv = 0.0f;  // (QMV_INDEXED_ROUTE: logit threadIdx.x of the token, loaded before the activation row)
    if constexpr (MODE == QMV_INDEXED_ROUTE) {
        const int li = (int)threadIdx.x < ix.n_experts ? (int)threadIdx.x : ix.n_experts - 1;
        lv = attn_load_early(ix.route_logits + (size_t)(m / ix.x_div) * ix.n_experts + li);
        xr = x + (size_t)(m / ix.x_div) * ix.ldx;
        if (ix.w2) n_split = ix.n_split;
    }
    constexpr bool IS_FUSED = MODE == QMV_FUSED;
    constexpr bool IS_GLU = MODE == QMV_GLU || MODE == QMV_GLU_RMS;
    constexpr bool RMS_CT = MODE == QMV_GLU_RMS;  // (norm, no second input)
    if constexpr (IS_FUSED || IS_GLU || MODE == QMV_FUSED_NOX) {
        const size_t xo = (size_t)m * ix.ldx;
        xr = x + xo;
        if constexpr (!RMS_CT)
            if (ix.x2) xr2 = ix.x2 + xo;
    }
    if constexpr (IS_GLU) W2 = ix.w2;  // (n_split stays N: wrow() reads gate rows)
    float* yr = y + (size_t)m * ldy;
    uint16_t* yh = reinterpret_cast<uint16_t*>(y) + (size_t)m * ldy;  // QMV_HALF
    const bool acc_out = (IS_FUSED || MODE == QMV_ATTN || MODE == QMV_FUSED_NOX) && ix.accumulate;
    auto store = [&](int r, float v) {
        if constexpr (MODE == QMV_HALF) yh[r] = f32_to_f16_rne(v);
        else yr[r] = v;
    };

    // 1. activation loads first (s_waitcnt vmcnt is in order: the quantize step
    //    then waits for these only), 2. first weight row, 3. quantize to LDS.
    // 256-element activation chunks of a row of SPL slots, per wavefront
    constexpr int CHUNKS = SPL * (64 / F::LPB) * F::ELEMS / QK_K;
    constexpr int MAXQ = (CHUNKS + NW - 1) / NW;
    // rows of more Q8K superblocks than the workgroup has wavefronts (K =
    // 11008 at 16 wavefronts: three rounds of the 64-lane quantize): 16 lanes
    // per superblock, four per wavefront, one round (q8.hpp, act16_*)
    // (plain row loads only: with the SwiGLU input or the RMS norm the per-lane
    // work of four times the elements on a quarter of the lanes measured slower)
    constexpr bool QUAD = F::ACT == GGML_Q8K && MAXQ >= QMV_QUAD_MIN_ROUNDS && MR == 1 &&
                          (MODE == QMV_PLAIN || MODE == QMV_FUSED_NOX);
    constexpr int MAXQ4 = (CHUNKS + 4 * NW - 1) / (4 * NW);
    ActRowPre16<QUAD ? MAXQ4 : 1> pre16;
    ActRowPre<MAXQ> pre;
    ActRowPre<(MR > 1 ? MAXQ : 1)> pre_more[(MR > 1 ? MR - 1 : 1)];  // (MR > 1: rows m+1 ..)
    AttnRowPre<MODE == QMV_ATTN ? MAXQ : 1> apre;
    int apos = 0;
    if constexpr (MODE == QMV_HALF)
        act_row_load_h<F::ACT, NW, MAXQ>(reinterpret_cast<const uint16_t*>(x) + (size_t)m * K, K, w, lane, pre);
    else if constexpr (MODE == QMV_ATTN) {
        apos = __float_as_int(attn_load_early(reinterpret_cast<const float*>(ix.attn_pos)));
        attn_row_load<NW, MAXQ>(x, ix.attn_nsplit, K, w, lane, apre);
    } else if constexpr (QUAD) {
        act16_row_load<NW, MAXQ4>(xr, K, w, lane, pre16);  // (plain and prologue-free modes only)
    } else if constexpr (MODE == QMV_PLAIN || MODE == QMV_FUSED_NOX || RMS_CT) {
        act_row_load<F::ACT, NW, MAXQ>(xr, K, w, lane, pre);
    } else if (xr2)
        act_row_load_swiglu<F::ACT, NW, MAXQ>(xr, xr2, K, w, lane, pre);
    else
        act_row_load<F::ACT, NW, MAXQ>(xr, K, w, lane, pre);
    if constexpr (MR > 1) {  // the workgroup's other rows (clamped into the rows; the extra ones never stored)
#pragma unroll
        for (int i = 1; i < MR; i++) {
            const int mi = m + i < ix.rows ? m + i : ix.rows - 1;
            act_row_load<F::ACT, NW, MAXQ>(x + (size_t)mi * K, K, w, lane, pre_more[i - 1]);
        }
    }
    // The RMS gains with the activation row, ahead of the weight rows (QMV_FUSED
    // and the compile-time norm modes).  Loaded after them (in the norm, as
    // the QMV_GLU mode still does), the norm waited for the first weight
    // rows' arrival as well: Q4_K 4096x4096 with the norm 5.28 -> 4.50 us,
    // 4096x8192 6.79 -> 6.21.  Without a norm (QMV_FUSED) these loads read
    // the activation row again and are never used.
    constexpr bool RMS_EARLY = (MODE == QMV_FUSED || RMS_CT) && !QUAD;
    ActRowPre<RMS_EARLY ? MAXQ : 1> gpre;
    if constexpr (RMS_EARLY)
        act_row_gain_load<F::ACT, NW, MAXQ>(RMS_CT || ix.rms_gain ? ix.rms_gain : xr, K, w, lane, gpre);
    __builtin_amdgcn_sched_barrier(0);  // the activation loads go out ahead of the weight loads
    // Every wavefront's activation loads go out before any weight row of the
    // workgroup is requested: a barrier between them, in the plain and fused
    // modes with rows quantized by 64 lanes.  Graph replays, weights rotated
    // over 1.2 GB: Q4_K 4096x4096 4.65 -> 3.93 us, 4096x11008 7.32 -> 6.70,
    // 4096x32000 14.70 -> 14.29; Q6_K 5.52 -> 5.09, 9.69 -> 9.30, 22.07 ->
    // 21.64; with the RMS norm 4096x4096 5.83 -> 5.41, 4096x8192 7.05 -> 6.83.
    // Measured and left out: the 16-lane quantize's rows (11008x4096 8.56 ->
    // 8.87 us: a 44 KB row does not stay in L2 between launches and arrives
    // from memory behind every CU's weight requests either way, so the
    // barrier only delays the weight stream), the silu input (10.44 -> 11.49
    // us at K = 11008), the GLU mode and the attention merge (unchanged).
    constexpr bool XBAR = !QUAD && MR == 1 && (MODE == QMV_PLAIN || IS_FUSED || MODE == QMV_FUSED_NOX);
    if constexpr (XBAR) {
        if (!xr2) __builtin_amdgcn_s_barrier();  // (uniform: no silu input)
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MODE == QMV_INDEXED_ROUTE) {
        // wavefront 0 runs the token's routing rounds (a serial chain: copies
        // in every wavefront would only compete for the SIMDs) while the
        // activation loads are in flight, and hands the picks to the others
        // through LDS; workgroups with blockIdx.x = 0 also store the launch
        // row's pick and its softmax weight
        const int E = ix.n_experts, topk = ix.x_div, slot = m % topk;
        if ((int)threadIdx.x < E) s_rt[threadIdx.x] = lv;
        __syncthreads();
        if (w == 0) {
            RouteRow<2> rrow;
#pragma unroll
            for (int i = 0; i < 2; i++) rrow.v[i] = s_rt[lane + 64 * i < E ? lane + 64 * i : E - 1];
            int id;
            float wv;
            route_topk<2>(rrow, E, topk, lane, id, wv);
            if (lane < topk) s_pick[lane] = id;
        }
        __syncthreads();
        const int sel = __builtin_amdgcn_readfirstlane(s_pick[slot]);
        if (bx == 0 && w == 0) {
            const float wv = route_softmax(lane < topk ? s_rt[s_pick[lane < topk ? lane : 0]] : 0.0f, topk, lane);
            if (lane == slot) {
                ix.route_ids[m] = sel;
                ix.route_w[m] = wv;
            }
        }
        const size_t eoff = (size_t)sel * ix.expert_bytes;
        W += eoff;
        if (ix.w2) W2 = ix.w2 + eoff;
    }
    // rows >= n_split live in the second matrix (row - n_split)
    auto wrow = [&](int r) { return r < n_split ? W + (size_t)r * row_bytes : W2 + (size_t)(r - n_split) * row_bytes; };
    typename F::Raw ra[SPL], rb[SPL];
    // Residual values y[r] of the accumulate epilogue.  In the modes without
    // a prologue (QMV_FUSED_NOX, QMV_ATTN) every call issues one vector load
    // per row (y[r], or the activation row's first element when there is no
    // residual): under a branch, the compiler's waits after the join counted
    // as if the load had not been issued, so the quantize waited for the
    // first weight row; and the first one, wave-uniform and ahead of every
    // store, became a scalar-cache load that the quantize's LDS wait then
    // waited for (Q4_K 4096x4096 with the residual add 4.46 -> 4.23 us).
    // With the RMS norm (QMV_FUSED) the extra load measured 0.15-0.2 us
    // slower, so there it stays a plain load under the branch.
    constexpr bool RES_VEC = MODE == QMV_ATTN || MODE == QMV_FUSED_NOX;
    auto ldres = [&](int r, float cur) -> float {
        if constexpr (RES_VEC) return attn_load_early(acc_out ? yr + r : xr);
        else return acc_out ? yr[r] : cur;
    };
    float resa = 0.0f, resb = 0.0f;
    static_assert(RPW == 1 || (SPL == 1 && 64 / F::LPB == 16), "row groups: one slot set of 16 blocks");
    constexpr int SB = (64 / F::LPB) / RPW;              // block slots per row of a group
    const int rsub = RPW > 1 ? gi / SB : 0;              // this lane's row within the group
    const int gb = RPW > 1 ? gi % SB : gi;               // and its first block slot
    {  // (every lane, unconditionally: a wavefront without rows loads the last row and never uses it)
        const int rr = RPW > 1 ? row * RPW + rsub : row;
        const int r0 = rr < N ? rr : N - 1;
        qmv_load_row<F, SPL>(wrow(r0), gb, c, KB, ra);
        if constexpr (IS_GLU && SPL <= 2) qmv_load_row<F, SPL>(W2 + (size_t)r0 * row_bytes, gb, c, KB, rb);
        resa = ldres(r0, resa);
    }
    if constexpr (MODE == QMV_ATTN) {
        __builtin_amdgcn_sched_barrier(0);  // the merge's waits come after the first row's loads are out
        attn_row_merge<NW, MAXQ>(apre, ix.attn_nsplit, apos >= 0 && apos < ix.attn_max_ctx, pre);
    }
    if constexpr ((IS_FUSED || IS_GLU) && !QUAD) {  // (16-lane rows take none of these modes)
        // rms_norm_last_dim (sum of squares over the whole row, spread over the
        // wavefronts) and the affine gain, before quantization
        if (RMS_CT || ix.rms_gain) {
            const auto bsum = [&](float v) { return block_sum_waves<NW>(v, s_red, w, lane); };
            if constexpr (RMS_EARLY)
                act_row_rms_norm<F::ACT, NW, MAXQ>(pre, gpre, ix.rms_eps, K, w, lane, bsum);
            else
                act_row_rms_norm<F::ACT, NW, MAXQ>(pre, ix.rms_gain, ix.rms_eps, K, w, lane, bsum);
        }
    }
    if constexpr (QUAD)
        act16_row_quantize<NW, MAXQ4>(pre16, K, s_qs, lay.qstride, s_d, s_bs, w, lane);
    else
        act_row_quantize<F::ACT, NW, MAXQ>(pre, K, s_qs, lay.qstride, s_d, s_bs, w, lane);
    if constexpr (MR > 1) {
#pragma unroll
        for (int i = 1; i < MR; i++) {
            uint8_t* b = smem + (size_t)i * lay.bytes;
            act_row_quantize<F::ACT, NW, MAXQ>(pre_more[i - 1], K, reinterpret_cast<int8_t*>(b), lay.qstride,
                                               reinterpret_cast<float*>(b + lay.off_d),
                                               reinterpret_cast<int16_t*>(b + lay.off_bs), w, lane);
        }
    }
    __syncthreads();
    // With one activation row the lane's activation slices are the same for
    // every weight row: the GLU ring (rows of one or two slots) and Q8_0 rows
    // of up to four slots read them from LDS once and keep them in registers
    // (GLU 4096x22016 11.80 -> 11.45 us, Q8_0 4096x4096 5.91 -> 5.76,
    // 2048x8192 5.90 -> 5.64).  Elsewhere it measured slower, the compiler
    // scheduling the rows' loads and waits differently around them (Q4_K
    // 4096x11008 6.65 -> 7.05 us, fused RMS 4096x8192 6.03 -> 6.87, Q6_K
    // 4096x32000 21.6 -> 22.4; rows of three slots twice as slow).
    constexpr bool XREG = MR == 1 && RPW == 1 &&
                          ((IS_GLU && SPL <= 2) || (F::BYTES == Q8_0_BYTES && SPL <= 4));
    typename F::Act xa[XREG ? SPL : 1];
    if constexpr (XREG) qmv_load_acts<F, SPL>(s_qs, lay.qstride, s_d, s_bs, gb, c, KB, xa);
    auto rowdot = [&](const typename F::Raw(&r)[SPL]) __attribute__((always_inline)) -> float {
        if constexpr (XREG) return qmv_row_x<F, SPL, RPW>(r, xa, gb, c, KB);
        else return qmv_row<F, SPL, RPW>(r, s_qs, lay.qstride, s_d, s_bs, gb, c, KB);
    };
    // a row's sums against every activation row of the workgroup, stored
    auto emit = [&](const typename F::Raw(&r)[SPL], int row, float res) __attribute__((always_inline)) {
        if constexpr (MR == 1) {
            const float t = rowdot(r);
            if (lane == 63) store(row, acc_out ? res + t : t);
        } else {
#pragma unroll
            for (int i = 0; i < MR; i++) {
                const uint8_t* b = smem + (size_t)i * lay.bytes;
                const float t = qmv_row<F, SPL>(r, reinterpret_cast<const int8_t*>(b), lay.qstride,
                                                reinterpret_cast<const float*>(b + lay.off_d),
                                                reinterpret_cast<const int16_t*>(b + lay.off_bs), gi, c, KB);
                if (lane == 63 && m + i < ix.rows) y[(size_t)(m + i) * ldy + row] = t;
            }
        }
    };

    if constexpr (IS_GLU && SPL <= 2) {
        // Two output rows in flight: the gate and up rows of the wavefront's
        // next row (rc, rd, or ra, rb) load while this row's pair is reduced
        // (the pair of the first row was requested before the quantize).
        // Measured at 4096x22016: 13.5-14.0 -> 12.9-13.0 us, decode +0.9%;
        // wider rows keep the one-row ring below (the four rows' registers
        // would halve occupancy or spill).
        typename F::Raw rc[SPL], rd[SPL];
        // The outputs are kept in lanes (the wavefront's k-th row in lane k)
        // and stored after the loop: with a store inside it, whose registers
        // the next rows' address arithmetic then reused, the compiler waited
        // for the store -- and so, the counter being in order, for the pair
        // whose loads were issued before it -- at the top of every
        // iteration, which left one pair in flight instead of two.  The
        // launcher splits the rows so that no wavefront has more than 64.
        if ((N - row + nw - 1) / nw > 64) {  // (never, by the launcher's split)
            for (int r = row; r < N; r += nw)
                if (lane == 63) store(r, __builtin_nanf(""));
            return;
        }
        float keep = 0.0f;
        int kept = 0;
        const int row0 = row;
        auto put = [&](float v) {
            const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
            keep = lane == kept ? t : keep;
            kept++;
        };
        while (row < N) {
            int nrow = row + nw;
            int lrow = nrow < N ? nrow : row;
            qmv_load_row<F, SPL>(W + (size_t)lrow * row_bytes, gi, c, KB, rc);
            qmv_load_row<F, SPL>(W2 + (size_t)lrow * row_bytes, gi, c, KB, rd);
            float tg = rowdot(ra);
            float tu = rowdot(rb);
            qmv_settle_row<F, SPL>(ra);
            qmv_settle_row<F, SPL>(rb);
            put(silu_mul(tg, tu));
            row = nrow;
            if (row >= N) {  // (the re-issued pair settled too: the exit joins the loop's back edge)
                qmv_settle_row<F, SPL>(rc);
                qmv_settle_row<F, SPL>(rd);
                break;
            }
            nrow = row + nw;
            lrow = nrow < N ? nrow : row;
            qmv_load_row<F, SPL>(W + (size_t)lrow * row_bytes, gi, c, KB, ra);
            qmv_load_row<F, SPL>(W2 + (size_t)lrow * row_bytes, gi, c, KB, rb);
            tg = rowdot(rc);
            tu = rowdot(rd);
            qmv_settle_row<F, SPL>(rc);
            qmv_settle_row<F, SPL>(rd);
            put(silu_mul(tg, tu));
            row = nrow;
        }
        if (lane < kept) store(row0 + lane * nw, keep);
        return;
    } else if constexpr (IS_GLU) {
        // The ring alternates gate row r (ra) and up row r (rb): the up row's
        // loads are in flight while the gate row is reduced, the next gate
        // row's while the up row is.
        while (row < N) {
            qmv_load_row<F, SPL>(W2 + (size_t)row * row_bytes, gi, c, KB, rb);
            const float tg = rowdot(ra);
            const int nrow = row + nw;
            const int lrow = nrow < N ? nrow : row;
            qmv_load_row<F, SPL>(W + (size_t)lrow * row_bytes, gi, c, KB, ra);
            const float tu = rowdot(rb);
            if (lane == 63) store(row, silu_mul(tg, tu));
            row = nrow;
        }
        return;
    }
    if constexpr (RPW > 1) {
        // the two-row ring below over groups of RPW rows; the segment's last
        // lane stores its row
        const int ng = (N + RPW - 1) / RPW;
        const bool seg_last = (lane & (64 / RPW - 1)) == 64 / RPW - 1;
        // (a wavefront's last group issues no further loads, as below: Q4_K
        // 2048x12288 5.16 -> 5.00 us, 768x2048 2.82 -> 2.77; the MoE layer
        // unchanged)
        auto finish = [&](const typename F::Raw(&r)[SPL], float res, int g) {
            const float t = rowdot(r);
            const int my = g * RPW + rsub;
            if (seg_last && my < N) store(my, acc_out ? res + t : t);
        };
        if (row >= ng) return;
        while (true) {
            int ngrp = row + nw;
            if (ngrp >= ng) {
                finish(ra, resa, row);
                return;
            }
            int lr = ngrp * RPW + rsub < N ? ngrp * RPW + rsub : N - 1;
            resb = ldres(lr, resb);
            qmv_load_row<F, SPL>(wrow(lr), gb, c, KB, rb);
            float t = rowdot(ra);
            int my = row * RPW + rsub;
            if (seg_last && my < N) store(my, acc_out ? resa + t : t);
            row = ngrp;
            ngrp = row + nw;
            if (ngrp >= ng) {
                finish(rb, resb, row);
                return;
            }
            lr = ngrp * RPW + rsub < N ? ngrp * RPW + rsub : N - 1;
            resa = ldres(lr, resa);
            qmv_load_row<F, SPL>(wrow(lr), gb, c, KB, ra);
            t = rowdot(rb);
            my = row * RPW + rsub;
            if (seg_last && my < N) store(my, acc_out ? resb + t : t);
            row = ngrp;
        }
    }
    // Two-row ring: the next row's loads are in flight while a row is
    // reduced.  A wavefront's last row issues no further loads (a
    // wave-uniform branch).  Re-issuing the last row instead (cache-resident,
    // no branch) measured slower, its loads holding the wavefront's end: Q8_0
    // 4096x4096 6.9 -> 6.0 us, Q4_K 11008x4096 8.4 -> 7.9, fused RMS Q4_K
    // 4096x4096 4.63 -> 4.36, the q|k + v pair 9.58 -> 9.23, Q6_K 5-8%.
    while (true) {
        int nrow = row + nw;
        if (nrow >= N) {
            if (row < N) emit(ra, row, resa);
            return;
        }
        resb = ldres(nrow, resb);
        qmv_load_row<F, SPL>(wrow(nrow), gi, c, KB, rb);
        emit(ra, row, resa);
        row = nrow;
        nrow = row + nw;
        if (nrow >= N) {
            emit(rb, row, resb);
            return;
        }
        resa = ldres(nrow, resa);
        qmv_load_row<F, SPL>(wrow(nrow), gi, c, KB, ra);
        emit(rb, row, resb);
        row = nrow;
    }
}

template <class F, int SPL, int WG, int MODE, int RPW = 1, int MR = 1>
__global__ __launch_bounds__(WG) void qmv_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                 float* __restrict__ y, int N, int K, int ldy, QmvOpts ix) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_red[WG / 64];
    if constexpr (MODE == QMV_INDEXED_ROUTE) {  // the token's logits and picks
        __shared__ __align__(16) float s_rt[QMV_ROUTE_MAX_EXPERTS];
        __shared__ int s_pick[QMV_ROUTE_MAX_EXPERTS];
        qmv_body<F, SPL, WG, MODE, RPW>(W, x, y, N, K, ldy, ix, blockIdx.x, gridDim.x, smem, s_red, s_rt, s_pick);
    } else {
        qmv_body<F, SPL, WG, MODE, RPW, MR>(W, x, y, N, K, ldy, ix, blockIdx.x, gridDim.x, smem, s_red);
    }
}

// Two matrices of the same activation rows in one launch: workgroups
// [0, gx1) compute y1 = W1 a(x) (format F1, N1 rows), the others y2 = W2 a(x).
template <class F1, class F2, int SPL, int WG>
__global__ __launch_bounds__(WG) void qmv_pair_kernel(const uint8_t* __restrict__ W1, float* __restrict__ y1, int N1,
                                                      int gx1, const uint8_t* __restrict__ W2, float* __restrict__ y2,
                                                      int N2, const float* __restrict__ x, int K, QmvOpts ix) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_red[WG / 64];
    if ((int)blockIdx.x < gx1)
        qmv_body<F1, SPL, WG, QMV_FUSED>(W1, x, y1, N1, K, N1, ix, blockIdx.x, gx1, smem, s_red);
    else
        qmv_body<F2, SPL, WG, QMV_FUSED>(W2, x, y2, N2, K, N2, ix, blockIdx.x - gx1, gridDim.x - gx1, smem, s_red);
}

namespace {

template <class F, int SPL, int WG, int MODE, int RPW = 1, int MR = 1>
hipError_t launch_qmv_wg(const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy, const QmvOpts& ix,
                         hipStream_t s, int num_cus) {
    constexpr int NW = WG / 64;
    static int occ = -1;  // resident workgroups per CU for this instantiation
    if (occ < 0) {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, qmv_kernel<F, SPL, WG, MODE, RPW, MR>, WG, 16384 * MR) !=
                hipSuccess ||
            o < 1)
            o = 1;
        occ = o;
    }
    const size_t lds = (size_t)MR * act_lds_layout(F::ACT, K, F::QSTRIDE).bytes;
    if (lds > 65536) return hipErrorInvalidValue;
    const int groups = (N + RPW - 1) / RPW;  // (rows, or groups of RPW rows)
    const int need = (groups + NW - 1) / NW;
    const int gy = (M + MR - 1) / MR;  // (MR activation rows per workgroup)
    int cap = num_cus * occ / (gy > 0 ? gy : 1);
    if (cap < 1) cap = 1;
    const int gx = need < cap ? need : cap;
    QmvOpts o = ix;
    o.rows = M;
    constexpr bool GLU = MODE == QMV_GLU || MODE == QMV_GLU_RMS;
    const int chunk = 64 * gx * NW;  // (the GLU ring keeps at most 64 rows a wavefront)
    if (GLU && N > chunk) {
        const size_t row_bytes = (size_t)(K / F::ELEMS) * F::BYTES;
        for (int r0 = 0; r0 < N; r0 += chunk) {
            QmvOpts oc = o;
            oc.w2 = o.w2 + (size_t)r0 * row_bytes;
            const int n = N - r0 < chunk ? N - r0 : chunk;
            hipLaunchKernelGGL((qmv_kernel<F, SPL, WG, MODE, RPW, MR>), dim3(gx, gy), dim3(WG), lds, s,
                               w + (size_t)r0 * row_bytes, x, y + r0, n, K, ldy, oc);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    hipLaunchKernelGGL((qmv_kernel<F, SPL, WG, MODE, RPW, MR>), dim3(gx, gy), dim3(WG), lds, s, w, x, y, N, K, ldy, o);
    return hipGetLastError();
}

template <class F, int SPL, int MODE>
hipError_t launch_qmv(const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy, const QmvOpts& ix,
                      hipStream_t s, int num_cus) {
    // (the GLU mode reduces two rows per output: at most 512 threads there)
    constexpr int WGN0 = qmv_wg<F, SPL>(), WGB0 = qmv_wg_big<F, SPL>();
    constexpr bool GLU = MODE == QMV_GLU || MODE == QMV_GLU_RMS;
    constexpr int WGN = GLU && WGN0 > 512 ? 512 : WGN0;
    constexpr int WGB = GLU && WGB0 > 512 ? 512 : WGB0;
    // short rows (at most 8 of a wavefront step's 16 block slots): 2 or 4 rows per step
    if constexpr (SPL == 1 && 64 / F::LPB == 16 && !GLU && MODE != QMV_ATTN) {
        const int KB = K / F::ELEMS;
        if (KB <= 4) return launch_qmv_wg<F, 1, WGN, MODE, 4>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        if (KB <= 8) return launch_qmv_wg<F, 1, WGN, MODE, 2>(w, x, y, M, N, K, ldy, ix, s, num_cus);
    }
    if (WGB != WGN && (size_t)N * (size_t)M <= (size_t)num_cus * (WGB / 64) * 2)
        return launch_qmv_wg<F, SPL, WGB, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
    return launch_qmv_wg<F, SPL, WGN, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
}

template <class F, int MODE>
hipError_t launch_fmt(const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy, const QmvOpts& ix,
                      hipStream_t s, int num_cus) {
    constexpr int BPW = 64 / F::LPB;
    const int KB = K / F::ELEMS;
    const int spl = (KB + BPW - 1) / BPW;
    switch (spl) {
        case 1: return launch_qmv<F, 1, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case 2: return launch_qmv<F, 2, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case 3: return launch_qmv<F, 3, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case 4: return launch_qmv<F, 4, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case 5: return launch_qmv<F, 5, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case 6: return launch_qmv<F, 6, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case 7: return launch_qmv<F, 7, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case 8: return launch_qmv<F, 8, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        default: return hipErrorInvalidValue;  // K beyond 8 slots: rejected by the host check
    }
}

// Plain mode with MR activation rows per workgroup (each weight row reduced
// against all of them while it is in registers).
template <class F, int MR>
hipError_t launch_multi_fmt(const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy, hipStream_t s,
                            int num_cus) {
    constexpr int BPW = 64 / F::LPB;
    const int spl = (K / F::ELEMS + BPW - 1) / BPW;
    const QmvOpts o{};
#define FRQ_MR(S)                                                                                                  \
    case S: {                                                                                                      \
        constexpr int WG = qmv_wg_big<F, S>();                                                                     \
        return launch_qmv_wg<F, S, WG, QMV_PLAIN, 1, MR>(w, x, y, M, N, K, ldy, o, s, num_cus);                     \
    }
    if constexpr (F::LPB == 2) {  // Q8_0 (K <= 4096: four slots; qmv_multi_supported)
        switch (spl) {
            FRQ_MR(4)
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (spl) {  // (K <= 4096: one slot; qmv_multi_supported)
            FRQ_MR(1)
            default: return hipErrorInvalidValue;
        }
    }
#undef FRQ_MR
}

template <int MODE>
hipError_t launch_dtype(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                        const QmvOpts& ix, hipStream_t s, int num_cus) {
    switch (dtype) {
        case GGML_Q4K: return launch_fmt<Q4K, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case GGML_Q6K: return launch_fmt<Q6K, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case GGML_Q8_0: return launch_fmt<Q80, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        default: return hipErrorInvalidValue;
    }
}

// The k-quant formats only (the compile-time norm modes).
template <int MODE>
hipError_t launch_dtype_kq(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                           const QmvOpts& ix, hipStream_t s, int num_cus) {
    switch (dtype) {
        case GGML_Q4K: return launch_fmt<Q4K, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        case GGML_Q6K: return launch_fmt<Q6K, MODE>(w, x, y, M, N, K, ldy, ix, s, num_cus);
        default: return hipErrorInvalidValue;
    }
}

template <class F1, class F2, int SPL>
hipError_t launch_pair_spl(const uint8_t* w1, float* y1, int n1, const uint8_t* w2, float* y2, int n2, const float* x,
                           int M, int K, const QmvOpts& o, hipStream_t s, int num_cus) {
    // (at most 512 threads: three such workgroups per CU keep more rows in
    // flight than one of 1024; measured on the 7B decode's q|k + v pair +1%)
    constexpr int WG1 = qmv_wg_big<F1, SPL>(), WG2 = qmv_wg_big<F2, SPL>();
    constexpr int WG12 = WG1 < WG2 ? WG1 : WG2;
    constexpr int WG = WG12 > 512 ? 512 : WG12;
    constexpr int NW = WG / 64;
    static int occ = -1;
    if (occ < 0) {
        int v = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, qmv_pair_kernel<F1, F2, SPL, WG>, WG, 16384) !=
                hipSuccess || v < 1)
            v = 1;
        occ = v;
    }
    const size_t lds1 = (size_t)act_lds_layout(F1::ACT, K, F1::QSTRIDE).bytes;
    const size_t lds2 = (size_t)act_lds_layout(F2::ACT, K, F2::QSTRIDE).bytes;
    const size_t lds = lds1 > lds2 ? lds1 : lds2;  // (each workgroup lays out its own format's row)
    if (lds > 65536) return hipErrorInvalidValue;
    // workgroups split in proportion to the bytes of the two matrices
    const double b1 = (double)n1 * F1::BYTES, b2 = (double)n2 * F2::BYTES;
    int total = num_cus * occ / (M > 0 ? M : 1);
    if (total < 2) total = 2;
    int gx1 = (int)(total * b1 / (b1 + b2) + 0.5);
    gx1 = gx1 < 1 ? 1 : gx1 > total - 1 ? total - 1 : gx1;
    int gx2 = total - gx1;
    const int need1 = (n1 + NW - 1) / NW, need2 = (n2 + NW - 1) / NW;
    gx1 = gx1 < need1 ? gx1 : need1;
    gx2 = gx2 < need2 ? gx2 : need2;
    hipLaunchKernelGGL((qmv_pair_kernel<F1, F2, SPL, WG>), dim3(gx1 + gx2, M), dim3(WG), lds, s, w1, y1, n1, gx1, w2,
                       y2, n2, x, K, o);
    return hipGetLastError();
}

template <class F1, class F2>
hipError_t launch_pair_fmt(const uint8_t* w1, float* y1, int n1, const uint8_t* w2, float* y2, int n2, const float* x,
                           int M, int K, const QmvOpts& o, hipStream_t s, int num_cus) {
    const int spl = (K / QK_K + 15) / 16;  // both formats: 4 lanes per superblock, 16 superblocks per wave step
    switch (spl) {
        case 1: return launch_pair_spl<F1, F2, 1>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
        case 2: return launch_pair_spl<F1, F2, 2>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
        case 3: return launch_pair_spl<F1, F2, 3>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
        case 4: return launch_pair_spl<F1, F2, 4>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool qmv_pair_supported(int dt1, int dt2, int K) {
    const bool kq1 = dt1 == GGML_Q4K || dt1 == GGML_Q6K, kq2 = dt2 == GGML_Q4K || dt2 == GGML_Q6K;
    return kq1 && kq2 && K % QK_K == 0 && K <= 4 * 16 * QK_K;
}

hipError_t launch_qmv_pair(int dt1, const uint8_t* w1, float* y1, int n1, int dt2, const uint8_t* w2, float* y2,
                           int n2, const float* x, int M, int K, const QmvOpts& o, hipStream_t s, int num_cus) {
    if (dt1 == GGML_Q4K && dt2 == GGML_Q6K) return launch_pair_fmt<Q4K, Q6K>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
    if (dt1 == GGML_Q4K && dt2 == GGML_Q4K) return launch_pair_fmt<Q4K, Q4K>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
    if (dt1 == GGML_Q6K && dt2 == GGML_Q4K) return launch_pair_fmt<Q6K, Q4K>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
    if (dt1 == GGML_Q6K && dt2 == GGML_Q6K) return launch_pair_fmt<Q6K, Q6K>(w1, y1, n1, w2, y2, n2, x, M, K, o, s, num_cus);
    return hipErrorInvalidValue;
}

hipError_t launch_qmv(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                      hipStream_t s, int num_cus) {
    return launch_dtype<QMV_PLAIN>(dtype, w, x, y, M, N, K, ldy, QmvOpts{}, s, num_cus);
}

bool qmv_multi_supported(int dtype, int M, int N, int K) {
    // measured against the skinny MFMA kernel (Q4_K / Q6_K): two rows win at
    // K = 4096 (4096x4096 7.5 -> 6.2 us, 4096x32000 25.7 -> 18.2 us), three or
    // four only on wide matrices (4096x32000 M = 4 27.2 -> 25.4 us, 4096x11008
    // 17.1 -> 13.1 us; at N = 4096 7.6 against 8.6 us); longer rows (one
    // register slot no longer holds a lane's blocks) and more rows lose
    if (!(dtype == GGML_Q4K || dtype == GGML_Q6K || dtype == GGML_Q8_0) || K % QK_K || K > 16 * QK_K) return false;
    if (dtype == GGML_Q8_0)  // (four slots exactly; 5-8 rows: two row groups, each reading the weights)
        return K == 16 * QK_K && M >= 2 && (M <= QMV_MULTI_MAX_ROWS || (M <= 2 * QMV_MULTI_MAX_ROWS && N >= 8192));
    return M == 2 || (M >= 3 && M <= QMV_MULTI_MAX_ROWS && N >= 8192);
}

hipError_t launch_qmv_multi(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                            hipStream_t s, int num_cus) {
    if (!qmv_multi_supported(dtype, M, N, K)) return hipErrorInvalidValue;
    if (dtype == GGML_Q8_0)
        return M <= 2 ? launch_multi_fmt<Q80, 2>(w, x, y, M, N, K, ldy, s, num_cus)
                      : launch_multi_fmt<Q80, 4>(w, x, y, M, N, K, ldy, s, num_cus);
    if (dtype == GGML_Q4K)
        return M <= 2 ? launch_multi_fmt<Q4K, 2>(w, x, y, M, N, K, ldy, s, num_cus)
                      : launch_multi_fmt<Q4K, 4>(w, x, y, M, N, K, ldy, s, num_cus);
    return M <= 2 ? launch_multi_fmt<Q6K, 2>(w, x, y, M, N, K, ldy, s, num_cus)
                  : launch_multi_fmt<Q6K, 4>(w, x, y, M, N, K, ldy, s, num_cus);
}

hipError_t launch_qmv_indexed(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                              const QmvOpts& ix, hipStream_t s, int num_cus) {
    return launch_dtype<QMV_INDEXED>(dtype, w, x, y, M, N, K, ldy, ix, s, num_cus);
}

hipError_t launch_qmv_indexed_route(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K,
                                    int ldy, const QmvOpts& ix, hipStream_t s, int num_cus) {
    if (ix.n_experts < 1 || ix.n_experts > QMV_ROUTE_MAX_EXPERTS || ix.x_div < 1 || ix.x_div > ix.n_experts)
        return hipErrorInvalidValue;
    return launch_dtype<QMV_INDEXED_ROUTE>(dtype, w, x, y, M, N, K, ldy, ix, s, num_cus);
}

hipError_t launch_qmv_half(int dtype, const uint8_t* w, const uint16_t* x, uint16_t* y, int M, int N, int K, int ldy,
                           hipStream_t s, int num_cus) {
    return launch_dtype<QMV_HALF>(dtype, w, reinterpret_cast<const float*>(x), reinterpret_cast<float*>(y), M, N, K,
                                  ldy, QmvOpts{}, s, num_cus);
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
        F::load_act(act.qs + (size_t)m * K, F::ACT == GGML_Q8K ? QK_K : QK8_0, act.d + (size_t)m * KBa,
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

hipError_t launch_qmv_fused(int dtype, const uint8_t* w, const float* x, float* y, int M, int N, int K, int ldy,
                            const QmvOpts& o, hipStream_t s, int num_cus) {
    if (!o.x2 && !o.rms_gain) return launch_dtype<QMV_FUSED_NOX>(dtype, w, x, y, M, N, K, ldy, o, s, num_cus);
    return launch_dtype<QMV_FUSED>(dtype, w, x, y, M, N, K, ldy, o, s, num_cus);
}

hipError_t launch_qmv_glu(int dtype, const uint8_t* w_gate, const uint8_t* w_up, const float* x, float* y, int M, int N,
                          int K, int ldy, const QmvOpts& o, hipStream_t s, int num_cus) {
    QmvOpts g = o;
    g.w2 = w_up;
    g.accumulate = 0;
    if (g.rms_gain && !g.x2 && dtype != GGML_Q8_0)
        return launch_dtype_kq<QMV_GLU_RMS>(dtype, w_gate, x, y, M, N, K, ldy, g, s, num_cus);
    return launch_dtype<QMV_GLU>(dtype, w_gate, x, y, M, N, K, ldy, g, s, num_cus);
}

hipError_t launch_qmv_attn(int dtype, const uint8_t* w, const float* part, float* y, int N, int K, const QmvOpts& o,
                           hipStream_t s, int num_cus) {
    if (K % QK_K || K % ATTN_HEAD_DIM || o.attn_nsplit < 1 || o.attn_nsplit > ATTN_MERGE_CHUNK)
        return hipErrorInvalidValue;
    return launch_dtype<QMV_ATTN>(dtype, w, part, y, 1, N, K, N, o, s, num_cus);
}

}  // namespace frq
