// Wave-level activation quantizers, bit-exact with BlockQ8K::from_float
// (k_quants.rs:2230-2267) and BlockQ8_0::from_float (k_quants.rs:629-658).
// One definition serves the standalone quantize kernels and the fused
// quantize+mat-vec kernels.  Translation units including this header are
// built with -ffp-contract=off: nothing here may fuse into an FMA.
#pragma once

#include "common.hpp"

namespace frq {

// Quantized values of one 256-element superblock held by a wavefront: lane l
// owns elements 4l..4l+3 (packed int8 in `packed`), `bsum` is the sum of its
// 16-element group (valid in every lane of the group), `d` the block scale.
struct Q8KWave {
    uint32_t packed;
    int bsum;
    float d;
};

// Wave64 max of non-negative floats (NaN operands ignored, as fmaxf does):
// DPP row steps leave each 16-lane row's max in its lanes, four readlanes
// combine the rows into a wave-uniform value.
__device__ __forceinline__ float wave_max_nonneg(float v) {
#define FRQ_DPP_MAX(ctrl) \
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false)))
    FRQ_DPP_MAX(0xB1);   // quad_perm [1,0,3,2]
    FRQ_DPP_MAX(0x4E);   // quad_perm [2,3,0,1]
    FRQ_DPP_MAX(0x141);  // row_half_mirror
    FRQ_DPP_MAX(0x140);  // row_mirror
#undef FRQ_DPP_MAX
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Sum over each aligned group of 4 lanes (every lane of the group gets it).
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    return v;
}

// One code of BlockQ8K::from_float: (iscale * x).round().min(127) as i8
// (k_quants.rs:2253) -- half-away rounding, the NaN of inf * 0 taken to 127
// by min (NaN-ignoring), -inf saturating to -128.  The argument is within
// 128 (1 + 2^-23) in magnitude unless it is infinite or NaN, so the two
// clamps and the conversion are the saturating cast exactly.  The rounding is
// v + copysign(0.49999997, v) (0.49999997 the float below 0.5) truncated by
// the conversion: the sum's truncation equals roundf(v) for every float with
// |v| <= 129 (checked over all of them), and infinities and NaN pass through
// the sum unchanged.
__device__ __forceinline__ int q8k_code(float v) {
    const float r = v + copysignf(0.49999997f, v);
    return (int)fmaxf(fminf(r, 127.0f), -128.0f);
}

__device__ __forceinline__ uint32_t pack_i8x4(const int* q) {
    return (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
           ((uint32_t)(q[3] & 0xff) << 24);
}

// `v` = elements 4*lane..4*lane+3 of the superblock, already loaded.
// The reference keeps the first element of largest |x| (strict '<' scan, so
// NaN and 0 never win): amax = max |x| ignoring NaN, then the first lane (by
// ballot) and first slot in it with |x| == amax supplies the signed value.
// Branch-free: the codes are formed for every superblock and an all-zero
// (amax == 0) one is replaced by zeros and d = 0 at the end.
__device__ __forceinline__ Q8KWave q8k_quantize_vals(const float4 v, int lane) {
    const float xv[4] = {v.x, v.y, v.z, v.w};
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) m = fmaxf(m, fabsf(xv[i]));
    const float amax = wave_max_nonneg(m);
    const bool zero = amax == 0.0f;
    float mine = 0.0f;
    bool has = false;
#pragma unroll
    for (int i = 3; i >= 0; i--) {
        const bool hit = fabsf(xv[i]) == amax;
        mine = hit ? xv[i] : mine;
        has = has || hit;
    }
    // (no lane at all only for an all-NaN superblock, amax = 0: lane 63 then)
    const unsigned long long ballot = __ballot(has) | (1ull << 63);
    const int first = __builtin_ctzll(ballot);
    const float bval = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), first));
    const float iscale = -128.0f / bval;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = q8k_code(iscale * xv[i]);
    Q8KWave r;
    r.bsum = zero ? 0 : quad_sum(q[0] + q[1] + q[2] + q[3]);
    r.packed = zero ? 0u : pack_i8x4(q);
    r.d = zero ? 0.0f : 1.0f / iscale;
    return r;
}

__device__ __forceinline__ Q8KWave q8k_quantize_wave(const float* __restrict__ x256, int lane) {
    return q8k_quantize_vals(reinterpret_cast<const float4*>(x256)[lane], lane);
}

// Eight 32-element blocks per wavefront: lane l owns elements 4(l%8).. of
// block l/8.  `live` lanes hold a real block.
struct Q80Wave {
    uint32_t packed;
    uint16_t dbits;
};

// `v` = elements 4*(lane%8).. of block lane/8 (zeros for lanes without a block).
__device__ __forceinline__ Q80Wave q8_0_quantize_vals(const float4 v, int lane) {
    const float xv[4] = {v.x, v.y, v.z, v.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(xv[i]));
    // max over the block's 8 lanes (an aligned half of a DPP row)
#define FRQ_DPP_MAX(ctrl) \
    amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, amax), ctrl, 0xF, 0xF, false)))
    FRQ_DPP_MAX(0xB1);   // quad_perm [1,0,3,2]
    FRQ_DPP_MAX(0x4E);   // quad_perm [2,3,0,1]
    FRQ_DPP_MAX(0x141);  // row_half_mirror: lane i <-> 7-i within each 8-lane half
#undef FRQ_DPP_MAX
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = sat_i8(roundf(xv[i] * id));
    Q80Wave r;
    r.packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
               ((uint32_t)(q[3] & 0xff) << 24);
    r.dbits = f32_to_f16_rne(d);
    return r;
}

__device__ __forceinline__ Q80Wave q8_0_quantize_wave(const float* __restrict__ x32, bool live, int lane) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v = reinterpret_cast<const float4*>(x32)[lane & 7];
    return q8_0_quantize_vals(v, lane);
}

// Quantize one activation row x[K] into an ActView row (qs / d / bsums) with
// the NW wavefronts of a workgroup.  The row is cut into 256-element chunks
// (one Q8K superblock, or eight Q8_0 blocks); wavefront w owns chunks
// w, w+NW, ..., at most MAXQ of them, and issues all their float4 loads
// (act_row_load) before any arithmetic (act_row_quantize), so the whole row
// costs one memory round trip.  The caller sizes MAXQ >= ceil(chunks / NW).
template <int MAXQ>
struct ActRowPre {
    float4 v[MAXQ];
};

// Lane `lane`'s four elements of chunk w + NW*i: live unless the chunk is past
// the row (or, for Q8_0 rows that end on a 32-element block, the lane is past
// K).  Every load is issued, from a clamped in-row offset, and nothing reads
// the registers before the quantize step: a load under a lane condition would
// make the compiler wait for it at once (to merge the zero and the loaded
// value), before the first weight rows are even requested.  Values of dead
// slots are never used unmasked.
template <int ACT>
__device__ __forceinline__ bool act_live(int ch, int nchunks, int K, int lane) {
    return ch < nchunks && (ACT == GGML_Q8K || ch * QK_K + 4 * lane < K);
}
__device__ __forceinline__ int act_elem(int ch, int nchunks, int K, int lane) {
    const int e = (ch < nchunks ? ch : nchunks - 1) * QK_K + 4 * lane;
    return e < K - 4 ? e : K - 4;
}

// A relaxed (workgroup-scope) atomic load is an ordinary global load on this
// target, but the compiler keeps it where it is written instead of sinking it
// to its first use, so the row's loads go out ahead of the weight loads.
__device__ __forceinline__ float4 load_f4_early(const float* p) {
    const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
    const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                       __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32)));
}

template <int ACT, int NW, int MAXQ>
__device__ __forceinline__ void act_row_load(const float* __restrict__ x, int K, int w, int lane,
                                             ActRowPre<MAXQ>& p) {
    const int nchunks = (K + QK_K - 1) / QK_K;
#pragma unroll
    for (int i = 0; i < MAXQ; i++) p.v[i] = load_f4_early(x + act_elem(w + NW * i, nchunks, K, lane));
}

// f16 activation row (matmul_f16, k_quants.rs:2333-2374): each half is
// widened exactly to f32 (half::f16::to_f32) before quantization.
template <int ACT, int NW, int MAXQ>
__device__ __forceinline__ void act_row_load_h(const uint16_t* __restrict__ x, int K, int w, int lane,
                                               ActRowPre<MAXQ>& p) {
    const int nchunks = (K + QK_K - 1) / QK_K;
    uint2 h[MAXQ];
#pragma unroll
    for (int i = 0; i < MAXQ; i++) h[i] = *reinterpret_cast<const uint2*>(x + act_elem(w + NW * i, nchunks, K, lane));
#pragma unroll
    for (int i = 0; i < MAXQ; i++)
        p.v[i] = make_float4(f16_to_f32(h[i].x & 0xffffu), f16_to_f32(h[i].x >> 16), f16_to_f32(h[i].y & 0xffffu),
                             f16_to_f32(h[i].y >> 16));
}

// SwiGLU input: silu(g) * u = g / (1 + exp(-g)) * u, element by element in the
// order of fuel's SiLU (byte_kernels.rs silu: x / (1 + (-x).exp())).
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int ACT, int NW, int MAXQ>
__device__ __forceinline__ void act_row_load_swiglu(const float* __restrict__ g, const float* __restrict__ u, int K,
                                                    int w, int lane, ActRowPre<MAXQ>& p) {
    ActRowPre<MAXQ> pu;
    act_row_load<ACT, NW, MAXQ>(g, K, w, lane, p);
    act_row_load<ACT, NW, MAXQ>(u, K, w, lane, pu);
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {
        p.v[i].x = silu_mul(p.v[i].x, pu.v[i].x);
        p.v[i].y = silu_mul(p.v[i].y, pu.v[i].y);
        p.v[i].z = silu_mul(p.v[i].z, pu.v[i].z);
        p.v[i].w = silu_mul(p.v[i].w, pu.v[i].w);
    }
}

// rms_norm_last_dim_f32 (fuel-cpu-backend/src/byte_kernels.rs:2339-2368) and
// the affine gain of apply_affine_rms_norm (fuel-core/src/lazy.rs:10330-10346)
// on a row held by the workgroup: y = (x * (1 / sqrt(sum(x^2) * (1/K) + eps)))
// * gain.  block_sum(v) sums one value per wavefront (lane 63) over the
// workgroup; the sum of squares is a tree here, sequential in the reference.
// `g` holds the gains of the lane's elements (act_row_gain_load, or the
// overload below that loads them itself).
template <int ACT, int NW, int MAXQ, class BlockSum>
__device__ __forceinline__ void act_row_rms_norm(ActRowPre<MAXQ>& p, const ActRowPre<MAXQ>& gp, float eps, int K,
                                                 int w, int lane, BlockSum block_sum) {
    const int nchunks = (K + QK_K - 1) / QK_K;
    const float4* g = gp.v;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {  // dead lanes / chunks count as zeros
        const float4 v = act_live<ACT>(w + NW * i, nchunks, K, lane) ? p.v[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    const float total = block_sum(dpp_wave_sum(ss));
    const float rinv = 1.0f / sqrtf(total * (1.0f / (float)K) + eps);
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {  // (dead slots are scaled too; they are never stored)
        p.v[i].x = (p.v[i].x * rinv) * g[i].x;
        p.v[i].y = (p.v[i].y * rinv) * g[i].y;
        p.v[i].z = (p.v[i].z * rinv) * g[i].z;
        p.v[i].w = (p.v[i].w * rinv) * g[i].w;
    }
}

// The gains of the lane's elements, loaded unconditionally like the row and,
// like it, as relaxed atomic loads: the compiler keeps them ahead of the
// weight rows' loads, so that the norm waits for the gains and the row only
// (the in-order vmcnt counter would otherwise make it wait for the first
// weight rows as well).
template <int ACT, int NW, int MAXQ>
__device__ __forceinline__ void act_row_gain_load(const float* __restrict__ gain, int K, int w, int lane,
                                                  ActRowPre<MAXQ>& g) {
    act_row_load<ACT, NW, MAXQ>(gain, K, w, lane, g);
}

template <int ACT, int NW, int MAXQ, class BlockSum>
__device__ __forceinline__ void act_row_rms_norm(ActRowPre<MAXQ>& p, const float* __restrict__ gain, float eps, int K,
                                                 int w, int lane, BlockSum block_sum) {
    const int nchunks = (K + QK_K - 1) / QK_K;
    ActRowPre<MAXQ> g;
#pragma unroll
    for (int i = 0; i < MAXQ; i++) g.v[i] = *reinterpret_cast<const float4*>(gain + act_elem(w + NW * i, nchunks, K, lane));
    act_row_rms_norm<ACT, NW, MAXQ>(p, g, eps, K, w, lane, block_sum);
}

// ---- Q8K rows with 16 lanes per superblock ----
// For long rows (more superblocks than a workgroup has wavefronts) the row is
// held four superblocks per wavefront: lanes 16g .. 16g+15 of wavefront w own
// superblock 4 (w + NW i) + g, lane t = l & 15 holding float4 j (j < 4) at
// elements 64 j + 4 t .. +3.  A load instruction (float4 j of every lane) then
// reads 256 contiguous bytes per superblock; with each lane's 16 elements
// contiguous instead (64 bytes a lane) every instruction touched four times
// the cache lines (11008x4096: 8.98 -> 8.66 us with this layout).  The
// maximum and the first index of the maximum are reduced within the 16-lane
// DPP row, with no readlanes; a 16-element bsum group is float4 j of four
// neighbouring lanes (a quad), summed exactly by two DPP steps.  The values
// are those of q8k_quantize_vals: the same maximum (order-free), the same
// first element (the smallest element index among the |x| == amax), the same
// iscale, rounding, saturation and d.
template <int MAXQ4>
struct ActRowPre16 {
    float4 v[MAXQ4][4];
};

template <int NW>
__device__ __forceinline__ int act16_chunk(int w, int i, int lane) {
    return 4 * (w + NW * i) + (lane >> 4);
}
// element offset of float4 j of lane `lane` in chunk ch (clamped into the row)
__device__ __forceinline__ int act16_elem(int ch, int nchunks, int lane, int j) {
    return (ch < nchunks ? ch : nchunks - 1) * QK_K + 64 * j + 4 * (lane & 15);
}

template <int NW, int MAXQ4>
__device__ __forceinline__ void act16_row_load(const float* __restrict__ x, int K, int w, int lane,
                                               ActRowPre16<MAXQ4>& p) {
    const int nchunks = K / QK_K;
#pragma unroll
    for (int i = 0; i < MAXQ4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) p.v[i][j] = load_f4_early(x + act16_elem(act16_chunk<NW>(w, i, lane), nchunks, lane, j));
}

template <int NW, int MAXQ4>
__device__ __forceinline__ void act16_row_load_swiglu(const float* __restrict__ g, const float* __restrict__ u, int K,
                                                      int w, int lane, ActRowPre16<MAXQ4>& p) {
    ActRowPre16<MAXQ4> pu;
    act16_row_load<NW, MAXQ4>(g, K, w, lane, p);
    act16_row_load<NW, MAXQ4>(u, K, w, lane, pu);
#pragma unroll
    for (int i = 0; i < MAXQ4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            p.v[i][j].x = silu_mul(p.v[i][j].x, pu.v[i][j].x);
            p.v[i][j].y = silu_mul(p.v[i][j].y, pu.v[i][j].y);
            p.v[i][j].z = silu_mul(p.v[i][j].z, pu.v[i][j].z);
            p.v[i][j].w = silu_mul(p.v[i][j].w, pu.v[i][j].w);
        }
}

// DPP steps over one 16-lane row (every lane of the row ends with the result)
__device__ __forceinline__ float row16_max(float v) {
#define FRQ_DPP_MAX(ctrl) \
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false)))
    FRQ_DPP_MAX(0xB1);   // quad_perm [1,0,3,2]
    FRQ_DPP_MAX(0x4E);   // quad_perm [2,3,0,1]
    FRQ_DPP_MAX(0x141);  // row_half_mirror
    FRQ_DPP_MAX(0x140);  // row_mirror
#undef FRQ_DPP_MAX
    return v;
}
__device__ __forceinline__ float row16_fmin(float v) {
#define FRQ_DPP_FMIN(ctrl) \
    v = fminf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false)))
    FRQ_DPP_FMIN(0xB1);
    FRQ_DPP_FMIN(0x4E);
    FRQ_DPP_FMIN(0x141);
    FRQ_DPP_FMIN(0x140);
#undef FRQ_DPP_FMIN
    return v;
}
__device__ __forceinline__ int row16_min(int v) {
#define FRQ_DPP_MIN(ctrl) v = min(v, __builtin_amdgcn_update_dpp(0, v, ctrl, 0xF, 0xF, false))
    FRQ_DPP_MIN(0xB1);
    FRQ_DPP_MIN(0x4E);
    FRQ_DPP_MIN(0x141);
    FRQ_DPP_MIN(0x140);
#undef FRQ_DPP_MIN
    return v;
}

// One superblock held by a 16-lane row: lane l16 owns float4 j at elements
// 64 j + 4 l16 .. +3.  Writes the lane's 16 quantized bytes, the bsums of its
// quad's four groups (lane 4a of the quad) and (lane 0 of the row) d into the
// LDS row at superblock ch.
__device__ __forceinline__ void q8k_quantize16_store(const float4 (&v)[4], int ch, int8_t* qs, int qstride, float* dv,
                                                     int16_t* bsums, int l16) {
    float xv[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        xv[4 * j] = v[j].x;
        xv[4 * j + 1] = v[j].y;
        xv[4 * j + 2] = v[j].z;
        xv[4 * j + 3] = v[j].w;
    }
    // largest and smallest element (NaN ignored, both against 0): the largest
    // |x| is the larger of pmax and -nmin, and it decides the signed value
    // unless +amax and -amax both occur
    float pmax = 0.0f, nmin = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        pmax = fmaxf(pmax, xv[e]);
        nmin = fminf(nmin, xv[e]);
    }
    pmax = row16_max(pmax);
    nmin = row16_fmin(nmin);
    const float amax = fmaxf(pmax, -nmin);
    const bool zero = amax == 0.0f;
    float bval = pmax > -nmin ? pmax : nmin;
    if (pmax == -nmin && !zero) {  // (uniform over the 16-lane row)
        // first element of |x| == amax: key = 2 * (element index) + sign bit,
        // minimized over the row (1023 when this lane has none); |x| == amax >
        // 0 makes x = +-amax exactly
        int key = 1023;
#pragma unroll
        for (int e = 15; e >= 0; e--) {  // (element index 64 (e / 4) + 4 l16 + e % 4 grows with e)
            const int k = 2 * (64 * (e >> 2) + 4 * l16 + (e & 3)) + (int)(__builtin_bit_cast(uint32_t, xv[e]) >> 31);
            key = fabsf(xv[e]) == amax ? k : key;
        }
        key = row16_min(key);
        bval = (key & 1) ? -amax : amax;
    }
    const float iscale = -128.0f / bval;
    int q[16];
#pragma unroll
    for (int e = 0; e < 16; e++) q[e] = q8k_code(iscale * xv[e]);
    int8_t* row = qs + (size_t)ch * qstride;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        *reinterpret_cast<uint32_t*>(row + 64 * j + 4 * l16) = zero ? 0u : pack_i8x4(q + 4 * j);
        // group 4 j + l16 / 4: float4 j of the quad's four lanes
        int g = q[4 * j] + q[4 * j + 1] + q[4 * j + 2] + q[4 * j + 3];
        g += __builtin_amdgcn_update_dpp(0, g, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
        g += __builtin_amdgcn_update_dpp(0, g, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
        if ((l16 & 3) == 0) bsums[ch * 16 + 4 * j + (l16 >> 2)] = (int16_t)(zero ? 0 : g);
    }
    if (l16 == 0) dv[ch] = zero ? 0.0f : 1.0f / iscale;
}

template <int NW, int MAXQ4>
__device__ __forceinline__ void act16_row_quantize(const ActRowPre16<MAXQ4>& p, int K, int8_t* qs, int qstride,
                                                   float* dv, int16_t* bsums, int w, int lane) {
    const int nchunks = K / QK_K;
#pragma unroll
    for (int i = 0; i < MAXQ4; i++) {
        const int ch = act16_chunk<NW>(w, i, lane);
        if (ch < nchunks) q8k_quantize16_store(p.v[i], ch, qs, qstride, dv, bsums, lane & 15);
    }
}

// Chunk `ch` (256 elements: one Q8K superblock or eight Q8_0 blocks) of an
// activation row of K elements, lane `lane` holding elements 4*lane.. of it.
template <int ACT>
__device__ __forceinline__ void act_chunk_quantize(const float4 v, int ch, int K, int8_t* qs, int qstride, float* dv,
                                                   int16_t* bsums, int lane) {
    if constexpr (ACT == GGML_Q8K) {
        const Q8KWave r = q8k_quantize_vals(v, lane);
        reinterpret_cast<uint32_t*>(qs + (size_t)ch * qstride)[lane] = r.packed;
        if ((lane & 3) == 0) bsums[ch * 16 + (lane >> 2)] = (int16_t)r.bsum;
        if (lane == 0) dv[ch] = r.d;
    } else {
        const Q80Wave r = q8_0_quantize_vals(v, lane);
        const int blk = ch * 8 + (lane >> 3);
        if (blk < K / QK8_0) {
            reinterpret_cast<uint32_t*>(qs + (size_t)blk * qstride)[lane & 7] = r.packed;
            if ((lane & 7) == 0) dv[blk] = f16_to_f32(r.dbits);
        }
    }
}

template <int ACT, int NW, int MAXQ>
__device__ __forceinline__ void act_row_quantize(const ActRowPre<MAXQ>& p, int K, int8_t* qs, int qstride,
                                                 float* dv, int16_t* bsums, int w, int lane) {
    const int nchunks = (K + QK_K - 1) / QK_K;
#pragma unroll
    for (int i = 0; i < MAXQ; i++) {
        const int ch = w + NW * i;
        if (ch >= nchunks) break;
        act_chunk_quantize<ACT>(p.v[i], ch, K, qs, qstride, dv, bsums, lane);
    }
}

}  // namespace frq
