// Top-k softmax routing of one token by one wavefront, shared by the routing
// kernel (moe.hip) and the gate|up mat-vec that routes its own token
// (mmvq.hip, QMV_INDEXED_ROUTE), so both produce the same ids and weights.
//
// Reference semantics: k rounds of argmax over the logits (first index on
// ties, byte_kernels.rs:8246-8261), each pick masked with += -1e30
// (fuel-core/src/lazy_nn/moe.rs:90-127), then a softmax over the picked
// original logits in pick order (fuel-inference/src/moe_routing.rs:252-275).
#pragma once

#include "common.hpp"

namespace frq {

// Element j = lane + 64 i of the token's E <= 64 * EPL logits.
template <int EPL>
struct RouteRow {
    float v[EPL];
};

template <int EPL>
__device__ __forceinline__ void route_load(const float* __restrict__ lr, int E, int lane, RouteRow<EPL>& r) {
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int j = lane + 64 * i;
        r.v[i] = __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(lr + (j < E ? j : E - 1)),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    }
}

// Softmax over the picked original logits in pick order: lane s < topk holds
// pick s's logit p; returns that lane's weight (moe_routing.rs:252-275: max
// by a scan in pick order, e^(p - max), the sum in pick order, times 1/sum).
__device__ __forceinline__ float route_softmax(float p, int topk, int lane) {
    auto lane_val = [](float x, int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
    };
    float mx = lane_val(p, 0);
    for (int s = 1; s < topk; s++) {
        const float ps = lane_val(p, s);
        if (ps > mx) mx = ps;
    }
    const float ex = lane < topk ? expf(p - mx) : 0.0f;
    float sum = 0.0f;
    for (int s = 0; s < topk; s++) sum += lane_val(ex, s);
    return ex * (1.0f / sum);
}

// Lane s < topk ends with pick s: its expert id and softmax weight.  The
// argmax keys are kept masked in place: key += -1e30 on a pick gives the key
// scan_key would give the masked logit (a finite logit stays finite, +-inf
// and NaN keys are unchanged by the addition, as scan_key of NaN + -1e30 is).
template <int EPL>
__device__ __forceinline__ void route_topk(const RouteRow<EPL>& row, int E, int topk, int lane, int& my_id,
                                           float& my_w) {
    float key[EPL];
    int idx[EPL];  // element index, or past every element for the empty slots
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int j = lane + 64 * i;
        key[i] = j < E ? scan_key(row.v[i], j) : -INFINITY;
        idx[i] = j < E ? j : 0x7fffffff;
    }
    my_id = 0;
    float my_val = 0.0f;  // the pick's original logit
    for (int s = 0; s < topk; s++) {
        float bv = key[0];
        int bi = idx[0];
#pragma unroll
        for (int i = 1; i < EPL; i++) argmax_merge(bv, bi, key[i], idx[i]);
        wave_argmax(bv, bi);  // (uniform: a real element always beats the empty slots)
        const int owner = bi & 63, slot = bi >> 6;
        float pv = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (slot == i)
                pv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, row.v[i]), owner));
        if (lane == s) {
            my_id = bi;
            my_val = pv;
        }
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (idx[i] == bi) key[i] += -1e30f;
    }
    my_w = route_softmax(lane < topk ? my_val : 0.0f, topk, lane);
}

}  // namespace frq
