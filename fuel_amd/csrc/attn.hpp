// Merge of the per-split decode-attention partials (flash-decoding), shared by
// attn_combine_kernel (decode.hip) and the attention-merging mat-vec
// (mmvq.hip) so that both produce the same bits.
//
// Split s of head h leaves o_s[HD] (unnormalized weighted values), m_s (its
// score maximum, -inf for an empty range) and l_s (sum of e^(score - m_s)) at
// part[(h * nsplit + s) * ATTN_PSTRIDE]: o at 0, m at HD, l at HD + 1.  The
// merged output is out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M),
// M = max_s m_s, computed ATTN_MERGE_CHUNK splits per step: M and the running
// sums are rescaled between steps, and with nsplit <= ATTN_MERGE_CHUNK it is
// the plain formula (one step, products summed in split order).  Split 0 is
// never empty, so M is finite after the first step.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace frq {

// One merge step over the splits s0 + c (c < ATTN_MERGE_CHUNK; a slot with
// s0 + c >= nsplit holds a repeated split and is dropped).  NE output
// elements share the head's (M, L).
template <int NE>
__device__ __forceinline__ void attn_merge_step(const float (&o)[ATTN_MERGE_CHUNK][NE], const float (&m)[ATTN_MERGE_CHUNK],
                                                const float (&l)[ATTN_MERGE_CHUNK], int s0, int nsplit, float& M,
                                                float& L, float (&O)[NE]) {
    float Mn = M;
#pragma unroll
    for (int c = 0; c < ATTN_MERGE_CHUNK; c++) Mn = fmaxf(Mn, s0 + c < nsplit ? m[c] : -__builtin_inff());
    if (Mn != M) {  // M = -inf only before the first step, where L = O = 0
        const float r = expf(M - Mn);
        L *= r;
#pragma unroll
        for (int e = 0; e < NE; e++) O[e] *= r;
        M = Mn;
    }
#pragma unroll
    for (int c = 0; c < ATTN_MERGE_CHUNK; c++) {
        // an empty range has max -inf: factor 0; a repeated split: factor 0
        const float f = s0 + c < nsplit ? expf(m[c] - M) : 0.0f;
        L = fmaf(l[c], f, L);
#pragma unroll
        for (int e = 0; e < NE; e++) O[e] = fmaf(o[c][e], f, O[e]);
    }
}

// A relaxed workgroup-scope atomic load is a plain global load here; the
// compiler keeps it where it is written instead of sinking it to its use.
__device__ __forceinline__ float attn_load_early(const float* p) {
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_WORKGROUP));
}

}  // namespace frq
