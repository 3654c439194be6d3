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

#include "common.hpp"
#include "kernels.hpp"

namespace frq {

namespace {

constexpr int ROUTE_WG = 256;  // one wavefront per token

template <int EPL>
__global__ __launch_bounds__(ROUTE_WG) void moe_route_kernel(const float* __restrict__ logits, int T, int E, int topk,
                                                            int* __restrict__ ids, float* __restrict__ wts) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (ROUTE_WG / 64) + (threadIdx.x >> 6);
    if (t >= T) return;  // whole wavefront
    const float* lr = logits + (size_t)t * E;
    float v[EPL], orig[EPL];  // element j = lane + 64 i (orig: as loaded, for the softmax)
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int j = lane + 64 * i;
        orig[i] = lr[j < E ? j : E - 1];
        v[i] = orig[i];
    }
    int my_id = 0;       // lane s < topk keeps the s-th pick
    float my_val = 0.0f; // and its original logit
    for (int s = 0; s < topk; s++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int j = lane + 64 * i;
            if (j < E) argmax_merge(bv, bi, scan_key(v[i], j), j);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            argmax_merge(bv, bi, ov, oi);
        }
        float pv = 0.0f;  // the pick's original logit, from its owner lane
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const float o = __shfl(orig[i], bi & 63);
            if ((bi >> 6) == i) pv = o;
        }
        if (lane == s) {
            my_id = bi;
            my_val = pv;
        }
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (lane + 64 * i == bi) v[i] += -1e30f;
    }
    // softmax over the picked (original) logits, in pick order
    const float p = lane < topk ? my_val : 0.0f;
    float mx = __shfl(p, 0);
    for (int s = 1; s < topk; s++) {
        const float ps = __shfl(p, s);
        if (ps > mx) mx = ps;
    }
    const float ex = lane < topk ? expf(p - mx) : 0.0f;
    float sum = 0.0f;
    for (int s = 0; s < topk; s++) sum += __shfl(ex, s);
    const float inv = 1.0f / sum;
    if (lane < topk) {
        ids[(size_t)t * topk + lane] = my_id;
        wts[(size_t)t * topk + lane] = ex * inv;
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

}  // namespace frq
