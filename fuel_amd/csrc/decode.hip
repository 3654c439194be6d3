// Decode-step kernels around the quantized mat-vecs of a LLaMA-shaped
// decoder (fuel-core/src/lazy.rs:7363-7440, one token at position pos):
//
//   attention: RoPE of q and k (rotate-half with the f32 tables of
//   build_rope_tables, fuel-graph/src/lib.rs:10808-10868; rope_f32,
//   fuel-cpu-backend/src/byte_kernels.rs:1885-1964), append of k and v to an
//   f16 KV cache, scores (q . k_j) * scale, softmax over j <= pos and the
//   weighted sum of the values, per head.  The context is split over
//   workgroups (flash-decoding); the splits are merged by a second kernel
//   here, or inside the o-projection mat-vec (mmvq.hip, QMV_ATTN).
//
//   argmax + embedding: the next token (the prompt's while it lasts, else the
//   first-index argmax of the logits, argmax_dim_f32 byte_kernels.rs:8246),
//   its embedding row into the residual stream, pos += 1.  Both read pos from
//   device memory so that a captured step replays for every token.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "attn.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace frq {

namespace {

constexpr int HD = ATTN_HEAD_DIM;
constexpr int ATT_WG = 512;
constexpr int GROUPS = ATT_WG / 16;  // positions in flight per workgroup (16 lanes each)
static_assert(HD == 128 && ATT_WG >= 2 * HD && ATT_WG % 64 == 0, "the rope / append stage maps HD/2 elements to each of waves 0..3");

// Sum over 16-lane groups, every lane of a group ending with it: the DPP
// row steps of dpp_seg_sum (plain VALU operations; measured against four
// __shfl_xor steps through the LDS crossbar: decode +1%; the prefill
// attention kernel keeps the shuffles, which measured faster there).
__device__ __forceinline__ float group16_sum(float v) { return dpp_seg_sum<4>(v); }

// Raw f16 x 8 chunk (one 16-byte load) to floats.
__device__ __forceinline__ void h8_to_f(const uint4& u, float (&f)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = __half2float(__ushort_as_half((unsigned short)(w[i] & 0xffffu)));
        f[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(w[i] >> 16)));
    }
}

// grid = (heads, nsplit), ATT_WG = 512 threads (two wavefronts per SIMD at one
// workgroup per CU; against 256 threads and twice the iterations: decode
// +0.8%).  qk = [q | k] unrotated (heads * HD each), vn = v; caches are
// [heads][max_ctx][HD] f16.  Split sp of a head
// takes a contiguous range of at most 32 * ATTN_NIT positions: 16 lanes per
// position (8 dims per lane), every K and V load of the range issued before
// any arithmetic (one memory round trip).  It writes its unnormalized output,
// max and sum to part[head][sp]; attn_combine_kernel merges the splits (a
// kernel boundary, not a device-scope fence, orders the two).
__global__ __launch_bounds__(ATT_WG) void attn_split_kernel(const float* __restrict__ qk, const float* __restrict__ vn,
                                                           const float* __restrict__ rcos,
                                                           const float* __restrict__ rsin, __half* kc, __half* vc,
                                                           int max_ctx, const int* __restrict__ pos_p, float scale,
                                                           float* __restrict__ part) {
    __shared__ float s_q[HD], s_kn[HD], s_vn[HD];
    __shared__ float s_acc[ATT_WG / 64][HD];
    __shared__ float s_red[ATT_WG / 64];
    const int h = blockIdx.x, sp = blockIdx.y, H = gridDim.x, nsplit = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = tid >> 4, l16 = tid & 15;
    // 1. the new row's inputs, issued before pos is known: wave 0 rotates q,
    // wave 1 rotates k (elements lane and lane + HD/2), waves 2 and 3 take
    // v's two halves (one element each; hi repeats lo's address there);
    // waves 4.. load wave 2's addresses and append nothing.
    const int w = __builtin_amdgcn_readfirstlane(wave);
    const float* xs = w == 0 ? qk + (size_t)h * HD
                             : (w == 1 ? qk + (size_t)(H + h) * HD : vn + (size_t)h * HD + (HD / 2) * (w == 3));
    const float x_lo = attn_load_early(xs + lane), x_hi = attn_load_early(xs + (w < 2 ? lane + HD / 2 : lane));
    const int pos = *pos_p;
    if (pos < 0 || pos >= max_ctx) return;  // the combine writes NaN
    const int n = pos + 1;
    const int chunk = (n + nsplit - 1) / nsplit;
    const int p0 = min(n, sp * chunk), p1 = min(n, p0 + chunk);
    const bool owner = p0 < p1 && p1 == n;  // this split holds the new position
    const size_t cbase = (size_t)h * max_ctx * HD;
    const float* cs = rcos + (size_t)pos * HD;
    const float* sn = rsin + (size_t)pos * HD;
    const float c_lo = cs[lane], c_hi = cs[lane + HD / 2], s_lo = sn[lane], s_hi = sn[lane + HD / 2];
    __builtin_amdgcn_sched_barrier(0);

    // 2. every K / V load of the range, from positions clamped into it (p1 >= 1
    // always: an empty range is [n, n)); slots past p1 are masked at use.  Row
    // pos is stale in memory and is replaced below.
    uint4 kr[ATTN_NIT], vr[ATTN_NIT];
#pragma unroll
    for (int it = 0; it < ATTN_NIT; it++) {
        const int j = min(p0 + g + GROUPS * it, p1 - 1);
        kr[it] = *reinterpret_cast<const uint4*>(kc + cbase + (size_t)j * HD + 8 * l16);
        vr[it] = *reinterpret_cast<const uint4*>(vc + cbase + (size_t)j * HD + 8 * l16);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. rope(q); in the owner split rope(k) and v, rounded to f16 and appended.
    // out[i] = x[i] cos[i] - x[i+h] sin[i], out[i+h] = x[i+h] cos[i+h] + x[i] sin[i+h]
    if (w == 0) {
        s_q[lane] = x_lo * c_lo - x_hi * s_lo;
        s_q[lane + HD / 2] = x_hi * c_hi + x_lo * s_hi;
    } else if (owner && w < 4) {  // (waves 4.. take no part in the append)
        if (w == 1) {
            const __half a = __float2half(x_lo * c_lo - x_hi * s_lo);
            const __half b = __float2half(x_hi * c_hi + x_lo * s_hi);
            kc[cbase + (size_t)pos * HD + lane] = a;
            kc[cbase + (size_t)pos * HD + lane + HD / 2] = b;
            s_kn[lane] = __half2float(a);
            s_kn[lane + HD / 2] = __half2float(b);
        } else {
            const int i = lane + (HD / 2) * (w - 2);
            const __half a = __float2half(x_lo);
            vc[cbase + (size_t)pos * HD + i] = a;
            s_vn[i] = __half2float(a);
        }
    }
    __syncthreads();

    // 4. scores (all 16 lanes of a group end with their position's score)
    float q8[8];
#pragma unroll
    for (int e = 0; e < 8; e++) q8[e] = s_q[8 * l16 + e];
    float sc[ATTN_NIT];
    float mx = -__builtin_inff();
#pragma unroll
    for (int it = 0; it < ATTN_NIT; it++) {
        const int j = p0 + g + GROUPS * it;
        float kv[8];
        h8_to_f(kr[it], kv);
        if (owner && j == pos) {  // (s_kn / s_vn hold data only in the owner split)
#pragma unroll
            for (int e = 0; e < 8; e++) kv[e] = s_kn[8 * l16 + e];
        }
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) d = fmaf(q8[e], kv[e], d);
        d = group16_sum(d) * scale;
        sc[it] = j < p1 ? d : -__builtin_inff();
        mx = fmaxf(mx, sc[it]);
    }
    // 5. softmax statistics of the range, weighted values
#pragma unroll
    for (int off = 32; off >= 16; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    mx = s_red[0];
#pragma unroll
    for (int w = 1; w < ATT_WG / 64; w++) mx = fmaxf(mx, s_red[w]);
    __syncthreads();
    float l = 0.0f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int it = 0; it < ATTN_NIT; it++) {
        const int j = p0 + g + GROUPS * it;
        const float p = j < p1 ? expf(sc[it] - mx) : 0.0f;
        l += p;
        float vv[8];
        h8_to_f(vr[it], vv);
        if (j >= p1) {  // a clamped slot (p is 0 there): keep stale rows out of the sum
#pragma unroll
            for (int e = 0; e < 8; e++) vv[e] = 0.0f;
        }
        if (owner && j == pos) {
#pragma unroll
            for (int e = 0; e < 8; e++) vv[e] = s_vn[8 * l16 + e];
        }
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = fmaf(p, vv[e], acc[e]);
    }
    // 6. sum over the 16 groups: in-wave across the 4 groups, then over waves
#pragma unroll
    for (int off = 32; off >= 16; off >>= 1) {
        l += __shfl_xor(l, off);
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] += __shfl_xor(acc[e], off);
    }
    if (lane < 16) {
#pragma unroll
        for (int e = 0; e < 8; e++) s_acc[wave][8 * l16 + e] = acc[e];
    }
    if (lane == 0) s_red[wave] = l;
    __syncthreads();
    float* pp = part + ((size_t)h * nsplit + sp) * ATTN_PSTRIDE;
    if (tid < HD) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < ATT_WG / 64; w++) o += s_acc[w][tid];
        pp[tid] = o;
    }
    if (tid == 0) {
        float lt = 0.0f;
#pragma unroll
        for (int w = 0; w < ATT_WG / 64; w++) lt += s_red[w];
        pp[HD] = mx;  // -inf for an empty range
        pp[HD + 1] = lt;
    }
}

// out[h] = the merge of the head's split partials (attn_merge_step, attn.hpp),
// one element per thread.  The partials of ATTN_MERGE_CHUNK splits are loaded
// together (clamped split index) so that a step is one memory round trip;
// pos is loaded first and checked by a select at the end: the partial loads
// do not wait for it.
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* __restrict__ part, int nsplit, int max_ctx,
                                                         const int* __restrict__ pos_p, float* __restrict__ out) {
    const int h = blockIdx.x, tid = threadIdx.x;
    const int pos = __float_as_int(attn_load_early(reinterpret_cast<const float*>(pos_p)));
    const float* ph = part + (size_t)h * nsplit * ATTN_PSTRIDE;
    float M = -__builtin_inff(), L = 0.0f, O[1] = {0.0f};
    for (int s0 = 0; s0 < nsplit; s0 += ATTN_MERGE_CHUNK) {
        float m[ATTN_MERGE_CHUNK], l[ATTN_MERGE_CHUNK], o[ATTN_MERGE_CHUNK][1];
#pragma unroll
        for (int c = 0; c < ATTN_MERGE_CHUNK; c++)
            o[c][0] = attn_load_early(ph + (size_t)min(s0 + c, nsplit - 1) * ATTN_PSTRIDE + tid);
#pragma unroll
        for (int c = 0; c < ATTN_MERGE_CHUNK; c++) {
            const float* q = ph + (size_t)min(s0 + c, nsplit - 1) * ATTN_PSTRIDE;
            m[c] = q[HD];
            l[c] = q[HD + 1];
        }
        attn_merge_step<1>(o, m, l, s0, nsplit, M, L, O);
    }
    out[(size_t)h * HD + tid] = (pos < 0 || pos >= max_ctx) ? __builtin_nanf("") : O[0] / L;
}

constexpr int AM_WG = 1024;
constexpr int AM_PER = 32;  // logits per thread and round: 32768 in flight at once

// One workgroup.  The logits of a round are all requested before any is
// compared (positions clamped into the vocabulary, the excess keyed out), and
// before pos is known, so the whole scan is one memory round trip for
// vocabularies up to AM_WG * AM_PER (a loop of dependent loads was 13.6 us).
__global__ __launch_bounds__(AM_WG) void argmax_embed_kernel(const float* __restrict__ logits, int vocab,
                                                            const float* __restrict__ table, int dim, int* tokens,
                                                            int tokens_cap, const int* prompt_len_p, int* pos_p,
                                                            float* __restrict__ x) {
    __shared__ float s_v[AM_WG / 64];
    __shared__ int s_i[AM_WG / 64];
    __shared__ int s_tok;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float lv[AM_PER];
#pragma unroll
    for (int u = 0; u < AM_PER; u++) lv[u] = attn_load_early(logits + min(tid + u * AM_WG, vocab - 1));
    const int pos = *pos_p;
    const int nxt = pos + 1;
    const bool forced = nxt < *prompt_len_p && nxt < tokens_cap;
    int tok;
    if (forced) {
        tok = tokens[nxt];
    } else {
        float bv = -__builtin_inff();
        int bi = 0x7fffffff;
        for (int i0 = 0; i0 < vocab; i0 += AM_WG * AM_PER) {
            if (i0) {
#pragma unroll
                for (int u = 0; u < AM_PER; u++) lv[u] = logits[min(i0 + tid + u * AM_WG, vocab - 1)];
            }
#pragma unroll
            for (int u = 0; u < AM_PER; u++) {
                const int i = i0 + tid + u * AM_WG;
                argmax_merge(bv, bi, i < vocab ? scan_key(lv[u], i) : -__builtin_inff(), i < vocab ? i : 0x7fffffff);
            }
        }
        wave_argmax(bv, bi);
        if (lane == 0) {
            s_v[wave] = bv;
            s_i[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < AM_WG / 64; w++) argmax_merge(bv, bi, s_v[w], s_i[w]);
            s_tok = bi;
        }
        __syncthreads();
        tok = s_tok;
    }
    if ((unsigned)tok >= (unsigned)vocab) tok = 0;  // an out-of-range prompt id reads row 0
    const float4* src = reinterpret_cast<const float4*>(table + (size_t)tok * dim);
    for (int i = tid; i < dim / 4; i += AM_WG) reinterpret_cast<float4*>(x)[i] = src[i];
    __syncthreads();  // every thread has read pos
    if (tid == 0) {
        if (!forced && nxt < tokens_cap) tokens[nxt] = tok;
        *pos_p = nxt;
    }
}

}  // namespace

int attn_decode_splits(int n_heads, int max_ctx) {
    int s = (256 + n_heads - 1) / n_heads;  // about one workgroup per CU in all
    const int need = (max_ctx + ATTN_MAX_CHUNK - 1) / ATTN_MAX_CHUNK;  // at most ATTN_MAX_CHUNK positions a split
    return s < need ? need : s;
}

size_t attn_decode_work_bytes(int n_heads, int max_ctx) {
    // the split partials, then room for the merged output (n_heads * HD) for
    // callers that merge into scratch (frq_attention_decode_oproj with many splits)
    return ((size_t)n_heads * attn_decode_splits(n_heads, max_ctx) * ATTN_PSTRIDE + (size_t)n_heads * HD) *
           sizeof(float);
}

hipError_t launch_attn_split(const float* qk, const float* v, const float* rcos, const float* rsin, uint16_t* kc,
                             uint16_t* vc, int n_heads, int max_ctx, const int* pos, float scale, float* part,
                             hipStream_t s) {
    const int ns = attn_decode_splits(n_heads, max_ctx);
    hipLaunchKernelGGL(attn_split_kernel, dim3(n_heads, ns), dim3(ATT_WG), 0, s, qk, v, rcos, rsin,
                       reinterpret_cast<__half*>(kc), reinterpret_cast<__half*>(vc), max_ctx, pos, scale, part);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const float* qk, const float* v, const float* rcos, const float* rsin, uint16_t* kc,
                              uint16_t* vc, int n_heads, int max_ctx, const int* pos, float scale, float* part,
                              float* out, hipStream_t s) {
    const hipError_t e = launch_attn_split(qk, v, rcos, rsin, kc, vc, n_heads, max_ctx, pos, scale, part, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(HD), 0, s, part, attn_decode_splits(n_heads, max_ctx),
                       max_ctx, pos, out);
    return hipGetLastError();
}

hipError_t launch_argmax_embed(const float* logits, int vocab, const float* table, int dim, int* tokens,
                               int tokens_cap, const int* prompt_len, int* pos, float* x, hipStream_t s) {
    hipLaunchKernelGGL(argmax_embed_kernel, dim3(1), dim3(AM_WG), 0, s, logits, vocab, table, dim, tokens, tokens_cap,
                       prompt_len, pos, x);
    return hipGetLastError();
}

}  // namespace frq
