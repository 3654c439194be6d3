// MoE mul_mat_id support on gfx950: top-k softmax routing of router logits,
// the expert batches of the routed (token, slot) entries, and the combine of
// the expert outputs back onto the tokens.  The expert projections themselves
// run through the indexed mat-vec (mmvq.hip) over the sorted entries.
//
// Reference semantics:
//   routing   fuel-core/src/lazy_nn/moe.rs:90-127 (k rounds of argmax, first
//             index on ties, byte_kernels.rs:8246-8261; the pick is masked
//             with += -1e30) and softmax over the picked logits
//             (fuel-inference/src/moe_routing.rs:252-275);
//   batches   moe_routing.rs:334-360 (experts ascending, entries in (token,
//             slot) order within an expert);
//   combine   lazy_nn/moe.rs:323-346 (out[t] += w_{t,e} * y_e[t] per expert in
//             ascending order, product then sum).
#include <hip/hip_runtime.h>

#include <atomic>

#include "attn.hpp"
#include "common.hpp"
#include "formats.hpp"
#include "kernels.hpp"
#include "q8.hpp"
#include "route.hpp"

namespace frq {

namespace {

constexpr int ROUTE_WG = 256;  // one wavefront per token

template <int EPL>
__global__ __launch_bounds__(ROUTE_WG) void moe_route_kernel(const float* __restrict__ logits, int T, int E, int topk,
                                                            int* __restrict__ ids, float* __restrict__ wts) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (ROUTE_WG / 64) + (threadIdx.x >> 6);
    if (t >= T) return;  // whole wavefront
    RouteRow<EPL> row;
    route_load<EPL>(logits + (size_t)t * E, E, lane, row);
    int id;
    float wv;
    route_topk<EPL>(row, E, topk, lane, id, wv);
    if (lane < topk) {
        ids[(size_t)t * topk + lane] = id;
        wts[(size_t)t * topk + lane] = wv;
    }
}

// ---- expert batches ----

constexpr int BATCH_WG = 1024;
constexpr int BATCH_WORDS = 4096;  // bitmap words per chunk, shared by the experts

__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(x, off);
        if (lane >= off) x += o;
    }
    return x;
}

// One workgroup: counts -> expert_offsets, then the entries in chunks.  Within
// a chunk every expert owns a bitmap over the chunk's entries; an entry's rank
// within its expert is the entries already placed by earlier chunks plus the
// set bits below it (prefix popcounts), which keeps (token, slot) order.
__global__ __launch_bounds__(BATCH_WG) void moe_batches_kernel(const int* __restrict__ ids, int P, int E, int topk,
                                                              int wpe, int* __restrict__ offsets,
                                                              int* __restrict__ sorted_token,
                                                              int* __restrict__ sorted_slot,
                                                              int* __restrict__ entry_expert,
                                                              int* __restrict__ entry_pos, MoeTiles tiles) {
    __shared__ int off[MOE_MAX_EXPERTS];
    __shared__ int fill[MOE_MAX_EXPERTS];
    __shared__ int tot[MOE_MAX_EXPERTS];
    __shared__ unsigned bits[BATCH_WORDS];
    __shared__ int pc[BATCH_WORDS];
    __shared__ int wsum[BATCH_WG / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    for (int e = tid; e < E; e += BATCH_WG) {
        off[e] = 0;
        fill[e] = 0;
    }
    __syncthreads();
    for (int i = tid; i < P; i += BATCH_WG) {
        const int e = ids[i];
        if ((unsigned)e < (unsigned)E) atomicAdd(&off[e], 1);
    }
    __syncthreads();
    // exclusive scan of the counts (E <= BATCH_WG: one per thread)
    const int c = tid < E ? off[tid] : 0;
    const int incl = wave_incl_scan(c, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; w++) base += wsum[w];
    const int excl = base + incl - c;
    if (tid < E) {
        off[tid] = excl;
        offsets[tid] = excl;
    }
    if (tid == E - 1) offsets[E] = excl + c;
    if (tiles.bm > 0) {  // tile table of the grouped matmul: ceil(count / bm) tiles per expert
        const int nt = (c + tiles.bm - 1) / tiles.bm;
        const int tincl = wave_incl_scan(nt, lane);
        __syncthreads();  // wsum of the count scan has been read
        if (lane == 63) wsum[wave] = tincl;
        __syncthreads();
        int tbase = 0;
        for (int w = 0; w < wave; w++) tbase += wsum[w];
        const int t0 = tbase + tincl - nt;
        for (int j = 0; j < nt; j++) {
            tiles.tile_expert[t0 + j] = tid;
            tiles.tile_row0[t0 + j] = excl + j * tiles.bm;
        }
        if (tid == E - 1) tiles.ntiles[0] = t0 + nt;
    }
    __syncthreads();

    const int chunk = 32 * wpe;
    for (int c0 = 0; c0 < P; c0 += chunk) {
        const int c1 = min(P, c0 + chunk);
        for (int i = tid; i < E * wpe; i += BATCH_WG) bits[i] = 0u;
        __syncthreads();
        for (int i = c0 + tid; i < c1; i += BATCH_WG) {
            const int e = ids[i];
            const int r = i - c0;
            if ((unsigned)e < (unsigned)E) atomicOr(&bits[e * wpe + (r >> 5)], 1u << (r & 31));
        }
        __syncthreads();
        for (int e = tid; e < E; e += BATCH_WG) {
            int run = 0;
            for (int k = 0; k < wpe; k++) {
                pc[e * wpe + k] = run;
                run += __popc(bits[e * wpe + k]);
            }
            tot[e] = run;
        }
        __syncthreads();
        for (int i = c0 + tid; i < c1; i += BATCH_WG) {
            const int e = ids[i];
            if ((unsigned)e >= (unsigned)E) continue;
            const int r = i - c0, wd = e * wpe + (r >> 5);
            const int rank = fill[e] + pc[wd] + __popc(bits[wd] & ((1u << (r & 31)) - 1u));
            const int pos = off[e] + rank;
            sorted_token[pos] = i / topk;
            if (sorted_slot) sorted_slot[pos] = i;
            entry_expert[pos] = e;
            entry_pos[i] = pos;
        }
        __syncthreads();
        for (int e = tid; e < E; e += BATCH_WG) fill[e] += tot[e];
        __syncthreads();
    }
}

// The same batches for E <= 256 experts, ranked with ballots instead of
// bitmaps (measured: 23-29 us -> a few us for 4096 entries).  The entries go in
// rounds of BATCH_NW * 64 * BATCH_G; wavefront w of a round takes BATCH_G
// consecutive 64-entry groups.  Within a group, the lanes holding an entry of
// the same expert are found by eight ballots over the id's bits (the lanes
// that agree on every bit), so an entry's rank among them is a popcount below
// its lane; the wavefront's running count per expert (LDS) turns that into a
// rank within the wavefront's share of the round.  Then, per expert, an
// exclusive prefix over the wavefronts (plus the earlier rounds' entries)
// places every entry: (round, wavefront, group, lane) is entry order, so
// (token, slot) order within an expert is kept, as build_expert_batches does.
constexpr int BATCH_NW = BATCH_WG / 64;
constexpr int BATCH_G = 4;
constexpr int BALLOT_MAX_EXPERTS = 256;

__global__ __launch_bounds__(BATCH_WG) void moe_batches_ballot_kernel(const int* __restrict__ ids, int P, int E,
                                                                     int topk, int* __restrict__ offsets,
                                                                     int* __restrict__ sorted_token,
                                                                     int* __restrict__ sorted_slot,
                                                                     int* __restrict__ entry_expert,
                                                                     int* __restrict__ entry_pos, MoeTiles tiles) {
    __shared__ int off[BALLOT_MAX_EXPERTS];
    __shared__ int fill[BALLOT_MAX_EXPERTS];
    __shared__ int wcnt[BATCH_NW][BALLOT_MAX_EXPERTS];
    __shared__ int wsum[BATCH_NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // counts -> expert_offsets (and the tile table), as moe_batches_kernel
    for (int e = tid; e < E; e += BATCH_WG) {
        off[e] = 0;
        fill[e] = 0;
    }
    __syncthreads();
    for (int i = tid; i < P; i += BATCH_WG) {
        const int e = ids[i];
        if ((unsigned)e < (unsigned)E) atomicAdd(&off[e], 1);
    }
    __syncthreads();
    const int c = tid < E ? off[tid] : 0;
    const int incl = wave_incl_scan(c, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; w++) base += wsum[w];
    const int excl = base + incl - c;
    if (tid < E) {
        off[tid] = excl;
        offsets[tid] = excl;
    }
    if (tid == E - 1) offsets[E] = excl + c;
    if (tiles.bm > 0) {
        const int nt = (c + tiles.bm - 1) / tiles.bm;
        const int tincl = wave_incl_scan(nt, lane);
        __syncthreads();
        if (lane == 63) wsum[wave] = tincl;
        __syncthreads();
        int tbase = 0;
        for (int w = 0; w < wave; w++) tbase += wsum[w];
        const int t0 = tbase + tincl - nt;
        for (int j = 0; j < nt; j++) {
            tiles.tile_expert[t0 + j] = tid;
            tiles.tile_row0[t0 + j] = excl + j * tiles.bm;
        }
        if (tid == E - 1) tiles.ntiles[0] = t0 + nt;
    }
    __syncthreads();

    const unsigned long long below = (1ull << lane) - 1ull;
    constexpr int ROUND = BATCH_NW * 64 * BATCH_G;
    for (int r0 = 0; r0 < P; r0 += ROUND) {
        for (int e = lane; e < E; e += 64) wcnt[wave][e] = 0;  // (this wavefront's row only)
        const int g0 = r0 + wave * 64 * BATCH_G;
        int ee[BATCH_G], rk[BATCH_G];
#pragma unroll
        for (int g = 0; g < BATCH_G; g++) {
            const int i = g0 + 64 * g + lane;
            const int e = i < P ? ids[i] : -1;
            const bool valid = (unsigned)e < (unsigned)E;
            unsigned long long m = __ballot(valid);
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const bool bit = (e >> b) & 1;
                const unsigned long long v = __ballot(bit);
                m &= bit ? v : ~v;
            }
            const int rank = __popcll(m & below);
            const int before = valid ? wcnt[wave][e] : 0;
            if (valid && rank == 0) wcnt[wave][e] = before + __popcll(m);
            ee[g] = valid ? e : -1;
            rk[g] = before + rank;
        }
        __syncthreads();
        for (int e = tid; e < E; e += BATCH_WG) {  // prefix over the wavefronts, after the earlier rounds
            int run = fill[e];
            for (int w = 0; w < BATCH_NW; w++) {
                const int cw = wcnt[w][e];
                wcnt[w][e] = run;
                run += cw;
            }
            fill[e] = run;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < BATCH_G; g++) {
            const int e = ee[g];
            if (e < 0) continue;
            const int i = g0 + 64 * g + lane;
            const int pos = off[e] + wcnt[wave][e] + rk[g];
            sorted_token[pos] = i / topk;
            if (sorted_slot) sorted_slot[pos] = i;
            entry_expert[pos] = e;
            entry_pos[i] = pos;
        }
        __syncthreads();
    }
}

// ---- combine ----

constexpr int COMBINE_WG = 256;

// out[t, :] = sum over the token's entries in ascending expert order (equal
// experts in slot order) of yd[pos, :] * w; the sum starts from 0.  pos is
// the entry's row in yd: entry_pos[t * topk + slot] (expert-sorted rows), or
// t * topk + slot when entry_pos is null (rows in routing order).
__global__ __launch_bounds__(COMBINE_WG) void moe_combine_kernel(const float* __restrict__ yd,
                                                                const int* __restrict__ ids,
                                                                const float* __restrict__ wts,
                                                                const int* __restrict__ entry_pos, int topk, int d,
                                                                float* __restrict__ out) {
    __shared__ int opos[MOE_MAX_TOPK];
    __shared__ float ow[MOE_MAX_TOPK];
    const int t = blockIdx.x, tid = threadIdx.x;
    if (tid < topk) {
        const int* ti = ids + (size_t)t * topk;
        const int e = ti[tid];
        int rank = 0;
        for (int s = 0; s < topk; s++) rank += ti[s] < e || (ti[s] == e && s < tid);
        opos[rank] = entry_pos ? entry_pos[(size_t)t * topk + tid] : t * topk + tid;
        ow[rank] = wts[(size_t)t * topk + tid];
    }
    __syncthreads();
    const int d4 = d >> 2;
    for (int c = blockIdx.y * COMBINE_WG + tid; c < d4; c += gridDim.y * COMBINE_WG) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int r = 0; r < topk; r++) {
            const float4 v = reinterpret_cast<const float4*>(yd + (size_t)opos[r] * d)[c];
            const float g = ow[r];
            acc.x = acc.x + v.x * g;
            acc.y = acc.y + v.y * g;
            acc.z = acc.z + v.z * g;
            acc.w = acc.w + v.w * g;
        }
        reinterpret_cast<float4*>(out + (size_t)t * d)[c] = acc;
    }
}

// ---- down projection + combine, few tokens ----

constexpr int DC_NW = 8;  // wavefronts per workgroup

template <int SEG>
__device__ __forceinline__ float seg_total(float v) {  // valid in the segment's last lane
    if constexpr (SEG == 16) return dpp_seg_sum<4>(v);
    else if constexpr (SEG == 32) return dpp_seg_sum<2>(v);
    else return dpp_wave_sum(v);
}

// out[t, n] = sum over token t's entries in ascending expert order (equal
// experts in slot order) of w * (W_e[n] . q8(silu(g) * u)), the sum starting
// from 0 with each product rounded before it is added: the indexed down
// mat-vec and moe_combine_kernel in one launch.  A workgroup quantizes the
// token's topk activation rows silu(g) * u (gu [P, 2 ffn], row t * topk +
// slot) into LDS; a wavefront takes output rows n with SEG lanes per entry
// (the entry's ffn / ELEMS blocks, LPB lanes each) and 64 / SEG entries per
// pass.  The combine order is worked out in registers from the token's ids
// (no LDS round trip), so the first row's weight loads go out before the
// activation quantize.  An expert id outside [0, E) gives a NaN product (its
// loads read expert 0).
template <class F, int SEG, int NPASS, int MAXQ>
__global__ __launch_bounds__(64 * DC_NW) void moe_down_combine_kernel(const uint8_t* __restrict__ W,
                                                                      size_t expert_bytes, int E,
                                                                      const float* __restrict__ gu,
                                                                      const int* __restrict__ ids,
                                                                      const float* __restrict__ wts, int topk,
                                                                      int ffn, int d, float* __restrict__ out) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int SPP = 64 / SEG;
    const int t = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const ActLds lay = act_lds_layout(F::ACT, ffn);
    const int abytes = align16i(lay.bytes);
    const int nch = (ffn + QK_K - 1) / QK_K;
    const int total = topk * nch;
    const float* gt = gu + (size_t)t * topk * 2 * ffn;

    // 1. the token's ids and weights (lane l < topk: entry l), then every
    //    activation load of the wavefront's chunks (entry s, chunk lc)
    const int li = lane < topk ? lane : topk - 1;
    const int my_e = __float_as_int(attn_load_early(reinterpret_cast<const float*>(ids + (size_t)t * topk + li)));
    const float my_w = attn_load_early(wts + (size_t)t * topk + li);
    float4 g[MAXQ], u[MAXQ];
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {
        const int c = w + DC_NW * i;
        const int cc = c < total ? c : total - 1;
        const int s = cc / nch, lc = cc - s * nch;
        const float* row = gt + (size_t)s * 2 * ffn + act_elem(lc, nch, ffn, lane);
        g[i] = load_f4_early(row);
        u[i] = load_f4_early(row + ffn);
    }
    // 2. combine order: entry l's rank among the token's entries (ascending
    //    expert, equal experts in slot order); rank r's entry by ballot
    int my_rank = 0;
    for (int s = 0; s < topk; s++) {
        const int es = __builtin_amdgcn_readlane(my_e, s);
        my_rank += es < my_e || (es == my_e && s < lane);
    }
    auto entry_of_rank = [&](int r) {  // r < topk, wave-uniform
        return (int)__builtin_ctzll(__ballot(lane < topk && my_rank == r));
    };
    const int seg = lane / SEG, sl = lane % SEG;
    const int KB = ffn / F::ELEMS;
    const size_t row_bytes = (size_t)KB * F::BYTES;
    const int gb = sl / F::LPB, c = sl % F::LPB;
    const int bl = gb < KB ? gb : KB - 1;
    int p_slot[NPASS], p_exp[NPASS];  // this lane's entry in each pass (its segment's rank)
#pragma unroll
    for (int q = 0; q < NPASS; q++) {
        int sl_q = 0;
#pragma unroll
        for (int j = 0; j < SPP; j++) {
            const int r = q * SPP + j;
            const int sj = entry_of_rank(r < topk ? r : topk - 1);
            if (seg == j) sl_q = sj;
        }
        p_slot[q] = sl_q;
        p_exp[q] = __builtin_amdgcn_ds_bpermute(4 * sl_q, my_e);
    }
    int n = blockIdx.x * DC_NW + w;
    auto load_row = [&](int nn, typename F::Raw(&raw)[NPASS]) {
#pragma unroll
        for (int q = 0; q < NPASS; q++) {
            const int ev = (unsigned)p_exp[q] < (unsigned)E ? p_exp[q] : 0;
            F::load(W + (size_t)ev * expert_bytes + (size_t)nn * row_bytes + (size_t)bl * F::BYTES, c, raw[q]);
        }
    };
    typename F::Raw raw[NPASS];
    load_row(n < d ? n : d - 1, raw);

    // 3. silu(g) * u, quantized into the entry's LDS row
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {
        const int cq = w + DC_NW * i;
        if (cq >= total) break;
        const int s = cq / nch, lc = cq - s * nch;
        const float4 v = make_float4(silu_mul(g[i].x, u[i].x), silu_mul(g[i].y, u[i].y), silu_mul(g[i].z, u[i].z),
                                     silu_mul(g[i].w, u[i].w));
        uint8_t* base = smem + (size_t)s * abytes;
        act_chunk_quantize<F::ACT>(v, lc, ffn, reinterpret_cast<int8_t*>(base), lay.qstride,
                                   reinterpret_cast<float*>(base + lay.off_d), reinterpret_cast<int16_t*>(base + lay.off_bs),
                                   lane);
    }
    __syncthreads();

    // 4. output rows, a two-row register ring: the next row's loads are in
    //    flight while a row is reduced; a wavefront's last row issues no
    //    further loads (a wave-uniform exit, as in the mat-vec rings)
    auto reduce_row = [&](int nn, const typename F::Raw(&rr)[NPASS]) {
        float y[NPASS];
#pragma unroll
        for (int q = 0; q < NPASS; q++) {
            const uint8_t* base = smem + (size_t)p_slot[q] * abytes;
            float acc = 0.0f;
            if (gb < KB) {
                typename F::Act xa;
                F::load_act(reinterpret_cast<const int8_t*>(base), lay.qstride,
                            reinterpret_cast<const float*>(base + lay.off_d),
                            reinterpret_cast<const int16_t*>(base + lay.off_bs), gb, c, xa);
                int isum, msum;
                float dw, dmw;
                F::dot(rr[q], xa, c, isum, msum, dw, dmw);
                acc = fmaf(dw * xa.d, (float)isum, acc);
                acc = fmaf(-(dmw * xa.d), (float)msum, acc);
            }
            y[q] = seg_total<SEG>(acc);
        }
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < NPASS; q++)
#pragma unroll
            for (int j = 0; j < SPP; j++) {
                const int r = q * SPP + j;
                if (r < topk) {
                    const int sr = entry_of_rank(r);
                    float yr = __builtin_bit_cast(float,
                                                  __builtin_amdgcn_readlane(__builtin_bit_cast(int, y[q]), j * SEG + SEG - 1));
                    if ((unsigned)__builtin_amdgcn_readlane(my_e, sr) >= (unsigned)E) yr = __builtin_nanf("");
                    const float wr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), sr));
                    o = o + yr * wr;
                }
            }
        if (lane == 0) out[(size_t)t * d + nn] = o;
    };
    const int stride = gridDim.x * DC_NW;
    typename F::Raw rb[NPASS];
    if (n >= d) return;
    while (true) {
        int nn = n + stride;
        if (nn >= d) {
            reduce_row(n, raw);
            return;
        }
        load_row(nn, rb);
        reduce_row(n, raw);
        n = nn;
        nn = n + stride;
        if (nn >= d) {
            reduce_row(n, rb);
            return;
        }
        load_row(nn, raw);
        reduce_row(n, rb);
        n = nn;
    }
}

// Launch shape of the fused down + combine: lanes per entry (SEG), passes
// (NPASS) and activation chunks per wavefront (MAXQ); false when the layer
// is outside what it is instantiated for.
struct DcShape {
    int seg, npass, maxq;
    size_t lds;
};

bool dc_shape(int dtype, int topk, int ffn, DcShape& sh) {
    int lpb, elems;
    if (dtype == GGML_Q4K || dtype == GGML_Q6K) {
        lpb = 4;
        elems = QK_K;
    } else if (dtype == GGML_Q8_0) {
        lpb = 2;
        elems = QK8_0;
    } else {
        return false;
    }
    if (topk < 1 || topk > MOE_MAX_TOPK || ffn < elems || ffn % elems) return false;
    const int lanes = lpb * (ffn / elems);
    sh.seg = lanes <= 16 ? 16 : lanes <= 32 ? 32 : 0;
    if (!sh.seg) return false;
    const int passes = (topk + 64 / sh.seg - 1) / (64 / sh.seg);
    sh.npass = passes <= 1 ? 1 : passes <= 2 ? 2 : passes <= 4 ? 4 : 0;
    const int q = (topk * ((ffn + QK_K - 1) / QK_K) + DC_NW - 1) / DC_NW;
    sh.maxq = q <= 1 ? 1 : q <= 2 ? 2 : q <= 4 ? 4 : 0;
    sh.lds = (size_t)topk * align16i(act_lds_layout(dtype == GGML_Q8_0 ? GGML_Q8_0 : GGML_Q8K, ffn).bytes);
    return sh.npass && sh.maxq && sh.lds <= 65536;
}

template <class F, int SEG, int NPASS, int MAXQ>
hipError_t launch_dc(const DcShape& sh, const uint8_t* w, size_t eb, int E, const float* gu, const int* ids,
                     const float* wts, int T, int topk, int ffn, int d, float* out, hipStream_t s, int num_cus) {
    // resident workgroups per CU at this launch's dynamic LDS size, cached per
    // instantiation and LDS size (lds << 16 | occupancy; the grid only spreads
    // whole output rows over workgroups, so it never changes a result)
    static std::atomic<long long> cached{-1};
    long long c = cached.load(std::memory_order_relaxed);
    int occ;
    if (c >= 0 && (c >> 16) == (long long)sh.lds) {
        occ = (int)(c & 0xffff);
    } else {
        int o = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, moe_down_combine_kernel<F, SEG, NPASS, MAXQ>, 64 * DC_NW,
                                                         sh.lds) != hipSuccess ||
            o < 1)
            o = 1;
        occ = o > 0xffff ? 0xffff : o;
        cached.store(((long long)sh.lds << 16) | occ, std::memory_order_relaxed);
    }
    const int need = (d + DC_NW - 1) / DC_NW;
    int cap = num_cus * occ / T;
    if (cap < 1) cap = 1;
    hipLaunchKernelGGL((moe_down_combine_kernel<F, SEG, NPASS, MAXQ>), dim3(need < cap ? need : cap, T),
                       dim3(64 * DC_NW), sh.lds, s, w, eb, E, gu, ids, wts, topk, ffn, d, out);
    return hipGetLastError();
}

template <class F, int SEG, int NPASS>
hipError_t launch_dc_q(const DcShape& sh, const uint8_t* w, size_t eb, int E, const float* gu, const int* ids,
                       const float* wts, int T, int topk, int ffn, int d, float* out, hipStream_t s, int num_cus) {
    switch (sh.maxq) {
        case 1: return launch_dc<F, SEG, NPASS, 1>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
        case 2: return launch_dc<F, SEG, NPASS, 2>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
        default: return launch_dc<F, SEG, NPASS, 4>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
    }
}

template <class F, int SEG>
hipError_t launch_dc_p(const DcShape& sh, const uint8_t* w, size_t eb, int E, const float* gu, const int* ids,
                       const float* wts, int T, int topk, int ffn, int d, float* out, hipStream_t s, int num_cus) {
    switch (sh.npass) {
        case 1: return launch_dc_q<F, SEG, 1>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
        case 2: return launch_dc_q<F, SEG, 2>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
        default: return launch_dc_q<F, SEG, 4>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
    }
}

template <class F>
hipError_t launch_dc_f(const DcShape& sh, const uint8_t* w, size_t eb, int E, const float* gu, const int* ids,
                       const float* wts, int T, int topk, int ffn, int d, float* out, hipStream_t s, int num_cus) {
    return sh.seg == 16 ? launch_dc_p<F, 16>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus)
                        : launch_dc_p<F, 32>(sh, w, eb, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
}

}  // namespace

hipError_t launch_moe_route(const float* logits, int T, int E, int topk, int* ids, float* w, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    const dim3 grid((T + ROUTE_WG / 64 - 1) / (ROUTE_WG / 64));
    if (E <= 64)
        hipLaunchKernelGGL(moe_route_kernel<1>, grid, dim3(ROUTE_WG), 0, s, logits, T, E, topk, ids, w);
    else if (E <= 128)
        hipLaunchKernelGGL(moe_route_kernel<2>, grid, dim3(ROUTE_WG), 0, s, logits, T, E, topk, ids, w);
    else if (E <= 256)
        hipLaunchKernelGGL(moe_route_kernel<4>, grid, dim3(ROUTE_WG), 0, s, logits, T, E, topk, ids, w);
    else if (E <= 512)
        hipLaunchKernelGGL(moe_route_kernel<8>, grid, dim3(ROUTE_WG), 0, s, logits, T, E, topk, ids, w);
    else if (E <= MOE_MAX_EXPERTS)
        hipLaunchKernelGGL(moe_route_kernel<16>, grid, dim3(ROUTE_WG), 0, s, logits, T, E, topk, ids, w);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_moe_batches(const int* ids, int P, int E, int topk, int* offsets, int* sorted_token,
                              int* sorted_slot, int* entry_expert, int* entry_pos, const MoeTiles& tiles,
                              hipStream_t s) {
    if (E <= 0 || E > MOE_MAX_EXPERTS || topk <= 0) return hipErrorInvalidValue;
    if (E <= BALLOT_MAX_EXPERTS) {
        hipLaunchKernelGGL(moe_batches_ballot_kernel, dim3(1), dim3(BATCH_WG), 0, s, ids, P, E, topk, offsets,
                           sorted_token, sorted_slot, entry_expert, entry_pos, tiles);
        return hipGetLastError();
    }
    // words per expert per chunk: enough for all P entries when they fit
    const int need = (P + 31) / 32;
    int wpe = BATCH_WORDS / E;
    if (need < wpe) wpe = need > 0 ? need : 1;
    hipLaunchKernelGGL(moe_batches_kernel, dim3(1), dim3(BATCH_WG), 0, s, ids, P, E, topk, wpe, offsets,
                       sorted_token, sorted_slot, entry_expert, entry_pos, tiles);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float* yd, const int* ids, const float* w, const int* entry_pos, int T, int topk,
                              int d, float* out, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    if (topk <= 0 || topk > MOE_MAX_TOPK || (d & 3)) return hipErrorInvalidValue;
    const int d4 = d / 4;
    const int gy = (d4 + COMBINE_WG - 1) / COMBINE_WG;
    hipLaunchKernelGGL(moe_combine_kernel, dim3(T, gy), dim3(COMBINE_WG), 0, s, yd, ids, w, entry_pos, topk, d, out);
    return hipGetLastError();
}

bool moe_down_combine_supported(int dtype, int topk, int ffn) {
    DcShape sh;
    return dc_shape(dtype, topk, ffn, sh);
}

hipError_t launch_moe_down_combine(int dtype, const uint8_t* w, size_t expert_bytes, int E, const float* gu,
                                   const int* ids, const float* wts, int T, int topk, int ffn, int d, float* out,
                                   hipStream_t s, int num_cus) {
    DcShape sh;
    if (!dc_shape(dtype, topk, ffn, sh) || T < 0 || d < 1) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    switch (dtype) {
        case GGML_Q4K: return launch_dc_f<Q4K>(sh, w, expert_bytes, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
        case GGML_Q6K: return launch_dc_f<Q6K>(sh, w, expert_bytes, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
        default: return launch_dc_f<Q80>(sh, w, expert_bytes, E, gu, ids, wts, T, topk, ffn, d, out, s, num_cus);
    }
}

}  // namespace frq
