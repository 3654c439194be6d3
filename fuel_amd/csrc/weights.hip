// Weight quantizers on the device (DynQuantizedStorage::quantize): f32 rows ->
// fuel's BlockQ4K / BlockQ6K / BlockQ8_0 bytes, bit-exact with from_float
// (k_quants.rs:1470-1528 with make_qkx1_quants utils.rs:229-286;
// k_quants.rs:2005-2075 with make_qx_quants utils.rs:62-226; k_quants.rs:629-658),
// and with from_float_imatrix for Q4_K and Q6_K (quantize_imatrix:
// k_quants.rs:1530-1593 with make_qkx3_quants utils.rs:358-469 and
// make_qp_quants utils.rs:472-563; k_quants.rs:2077-2145).
// One thread per superblock runs the reference's sequential float search in the
// same operation order (built with -ffp-contract=off; '/' is IEEE-correct).
//
// Also the synthetic-input generator: Philox-4x32-10 words
// (fuel-cpu-kernels/src/philox.rs:47-135) and a Box-Muller normal transform.
#include "common.hpp"
#include "kernels.hpp"
#include "q8.hpp"

namespace frq {

namespace {

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// f32::total_cmp key
__device__ __forceinline__ int total_key(float f) {
    const int b = __builtin_bit_cast(int, f);
    return b ^ (int)(((unsigned)(b >> 31)) >> 1);
}

// make_qkx1_quants(nmax = 15, ntry = 5, x[32]) -> (scale, -min)
__device__ void make_qkx1_quants_15_5(const float (&x)[32], float& out_scale, float& out_min) {
    float mn = x[0], mx = x[0];
    int kmn = total_key(x[0]), kmx = kmn;
#pragma unroll
    for (int i = 1; i < 32; i++) {
        const int k = total_key(x[i]);
        if (k < kmn) { kmn = k; mn = x[i]; }   // min_by: first minimum
        if (k >= kmx) { kmx = k; mx = x[i]; }  // max_by: last maximum
    }
    if (mx == mn) {
        out_scale = 0.0f;
        out_min = 0.0f;
        return;
    }
    float min = fminf(mn, 0.0f);
    float iscale = 15.0f / (mx - min);
    float scale = 1.0f / iscale;
    uint32_t l[4] = {0u, 0u, 0u, 0u};  // 32 nibbles
    for (int t = 0; t < 5; t++) {
        float sumlx = 0.0f;
        int suml2 = 0;
        bool changed = false;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int li = clampi(nearest_int(iscale * (x[i] - min)), 0, 15);
            const uint32_t old = (l[i >> 3] >> (4 * (i & 7))) & 0xfu;
            if ((uint32_t)li != old) {
                l[i >> 3] = (l[i >> 3] & ~(0xfu << (4 * (i & 7)))) | ((uint32_t)li << (4 * (i & 7)));
                changed = true;
            }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) sum += x[i] - scale * (float)((l[i >> 3] >> (4 * (i & 7))) & 0xfu);
        min = sum / 32.0f;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!changed) break;
    }
    out_scale = scale;
    out_min = -min;
}

__device__ __forceinline__ void load32(const float* p, float (&x)[32]) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = reinterpret_cast<const float4*>(p)[i];
        x[4 * i] = v.x;
        x[4 * i + 1] = v.y;
        x[4 * i + 2] = v.z;
        x[4 * i + 3] = v.w;
    }
}

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t (&q)[12], int& d, int& m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// make_qx_quants(n = 16, nmax = 32, rmse_type = 1, qw); ls gets l + 32.  The
// weights are qw (importance weights) or, with qw null, x * x.
__device__ float make_qx_quants_16(const float (&x)[16], int (&ls)[16], const float* __restrict__ qw) {
    float max = 0.0f, amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax == 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; i++) ls[i] = 0;
        return 0.0f;
    }
    const float iscale = -32.0f / max;
    float sumlx = 0.0f, suml2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int l = clampi(nearest_int(iscale * x[i]), -32, 31);
        ls[i] = l + 32;
        const float w = qw ? qw[i] : x[i] * x[i];
        const float lf = (float)l;
        sumlx += w * x[i] * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        const float is2 = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        bool changed = false;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int l = clampi(nearest_int(is2 * x[i]), -32, 31);
            if (l + 32 != ls[i]) changed = true;
            const float w = qw ? qw[i] : x[i] * x[i];
            const float lf = (float)l;
            slx += w * x[i] * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
#pragma unroll
        for (int i = 0; i < 16; i++) ls[i] = 32 + clampi(nearest_int(is2 * x[i]), -32, 31);
        sumlx = slx;
        suml2 = sl2;
        scale = sumlx / suml2;
        best = scale * sumlx;
    }
    for (int itry = 0; itry < 5; itry++) {
        int n_changed = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float w = qw ? qw[i] : x[i] * x[i];
            const int l = ls[i] - 32;
            float slx = sumlx - w * x[i] * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                const int new_l = clampi(nearest_int(x[i] * sl2 / slx), -32, 31);
                if (new_l != l) {
                    slx += w * x[i] * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        ls[i] = 32 + new_l;
                        sumlx = slx;
                        suml2 = sl2;
                        scale = sumlx / suml2;
                        best = scale * sumlx;
                        n_changed++;
                    }
                }
            }
        }
        if (n_changed == 0) break;
    }
    return scale;
}

// d, dmin, the packed scales and the 4-bit codes of one Q4_K superblock
// (k_quants.rs:1511-1527, also the tail of from_float_imatrix).
__device__ void q4k_store(const float* __restrict__ xb, const uint8_t (&sc)[12], uint16_t dh, uint16_t mh,
                          uint8_t* __restrict__ ob) {
    const float df = f16_to_f32(dh), mf = f16_to_f32(mh);
    uint32_t hdr[4];
    hdr[0] = (uint32_t)dh | ((uint32_t)mh << 16);
    hdr[1] = (uint32_t)sc[0] | ((uint32_t)sc[1] << 8) | ((uint32_t)sc[2] << 16) | ((uint32_t)sc[3] << 24);
    hdr[2] = (uint32_t)sc[4] | ((uint32_t)sc[5] << 8) | ((uint32_t)sc[6] << 16) | ((uint32_t)sc[7] << 24);
    hdr[3] = (uint32_t)sc[8] | ((uint32_t)sc[9] << 8) | ((uint32_t)sc[10] << 16) | ((uint32_t)sc[11] << 24);
    *reinterpret_cast<uint4*>(ob) = uint4{hdr[0], hdr[1], hdr[2], hdr[3]};
    for (int c = 0; c < 4; c++) {
        uint32_t words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int half = 0; half < 2; half++) {
            const int j = 2 * c + half;
            int s, m;
            scale_min_k4(j, sc, s, m);
            const float d = df * (float)s;
            if (d == 0.0f) continue;  // L stays 0
            const float dm = mf * (float)m;
            float v[32];
            load32(xb + 32 * j, v);
#pragma unroll
            for (int l = 0; l < 32; l++) {
                const int lv = clampi(nearest_int((v[l] + dm) / d), 0, 15);
                words[l >> 2] |= (uint32_t)lv << (8 * (l & 3) + 4 * half);
            }
        }
        uint4* dst = reinterpret_cast<uint4*>(ob + 16 + 32 * c);
        dst[0] = uint4{words[0], words[1], words[2], words[3]};
        dst[1] = uint4{words[4], words[5], words[6], words[7]};
    }
}

// make_qkx3_quants(nmax = 15, x[32], Some(w), rmin = -0.9, rdelta = 0.05,
// nstep = 36, use_mad = false) -> (scale, -min): the weighted least-squares
// (scale, min) over 38 candidate code sets, kept only when strictly better.
__device__ void make_qkx3_quants_15(const float (&x)[32], const float (&w)[32], float& out_scale,
                                    float& out_neg_min) {
    float min_val = x[0], max_val = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < 32; i++) {
        if (x[i] < min_val) min_val = x[i];
        if (x[i] > max_val) max_val = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (min_val > 0.0f) min_val = 0.0f;
    if (max_val <= min_val) {
        out_scale = 0.0f;
        out_neg_min = -min_val;
        return;
    }
    float iscale = 15.0f / (max_val - min_val);
    float scale = 1.0f / iscale;
    float best_mad = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int l = clampi(nearest_int(iscale * (x[i] - min_val)), 0, 15);
        float diff = scale * (float)l + min_val - x[i];
        diff = diff * diff;
        best_mad += w[i] * diff;
    }
    for (int is = 0; is <= 36; is++) {
        iscale = (-0.9f + 0.05f * (float)is + 15.0f) / (max_val - min_val);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        uint32_t la[4] = {0u, 0u, 0u, 0u};  // 32 nibbles
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int l = clampi(nearest_int(iscale * (x[i] - min_val)), 0, 15);
            la[i >> 3] |= (uint32_t)l << (4 * (i & 7));
            sum_l += w[i] * (float)l;
            sum_l2 += w[i] * ((float)l * (float)l);
            sum_xl += w[i] * (float)l * x[i];
        }
        const float d = sum_w * sum_l2 - sum_l * sum_l;
        if (d > 0.0f) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / d;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / d;
            if (this_min > 0.0f) {
                this_min = 0.0f;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) {
                float diff = this_scale * (float)((la[i >> 3] >> (4 * (i & 7))) & 0xfu) + this_min - x[i];
                diff = diff * diff;
                mad += w[i] * diff;
            }
            if (mad < best_mad) {  // (later candidates are cut from the accepted min)
                best_mad = mad;
                scale = this_scale;
                min_val = this_min;
            }
        }
    }
    out_scale = scale;
    out_neg_min = -min_val;
}

// Rust `f as u8`: saturating, NaN -> 0.
__device__ __forceinline__ int sat_u8f(float v) { return v != v || v <= 0.0f ? 0 : (v >= 255.0f ? 255 : (int)v); }

// make_qp_quants(n = 8, nmax = 63, x, l, qw) -> scale (l: codes 0..63).
__device__ float make_qp_quants_8(const float (&x)[8], int (&l)[8], const float (&qw)[8]) {
    float max = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) max = fmaxf(max, x[i]);
    if (max == 0.0f) {
#pragma unroll
        for (int i = 0; i < 8; i++) l[i] = 0;
        return 0.0f;
    }
    float iscale = 63.0f / max;
#pragma unroll
    for (int i = 0; i < 8; i++) l[i] = nearest_int(iscale * x[i]) & 0xff;  // i32 as u8
    const float scale = 1.0f / iscale;
    float best_mse = -0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float diff = x[i] - scale * (float)l[i];
        best_mse += qw[i] * diff * diff;
    }
    for (int is = -4; is <= 4; is++) {
        if (is == 0) continue;
        const float iscale_is = (0.1f * (float)is + 63.0f) / max;
        const float scale_is = 1.0f / iscale_is;
        float mse = -0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int li = nearest_int(iscale_is * x[i]) & 0xff;
            li = li < 63 ? li : 63;
            const float diff = x[i] - scale_is * (float)li;
            mse += qw[i] * diff * diff;
        }
        if (mse < best_mse) {
            best_mse = mse;
            iscale = iscale_is;
        }
    }
    float sumlx = 0.0f, suml2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int li = sat_u8f(roundf(iscale * x[i]));
        li = li < 63 ? li : 63;
        l[i] = li;
        sumlx += qw[i] * x[i] * (float)li;
        suml2 += qw[i] * ((float)li * (float)li);
    }
    for (int it = 0; it < 5; it++) {
        int n_changed = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float slx = sumlx - qw[i] * x[i] * (float)l[i];
            float sl2 = suml2 - qw[i] * ((float)l[i] * (float)l[i]);
            if (slx > 0.0f && sl2 > 0.0f) {
                int new_li = nearest_int(x[i] * sl2 / slx) & 0xff;
                new_li = new_li < 63 ? new_li : 63;
                if (new_li != l[i]) {
                    slx += qw[i] * x[i] * (float)new_li;
                    sl2 += qw[i] * ((float)new_li * (float)new_li);
                    if (slx * slx * suml2 > sumlx * sumlx * sl2) {
                        l[i] = new_li;
                        sumlx = slx;
                        suml2 = sl2;
                        n_changed++;
                    }
                }
            }
        }
        if (n_changed == 0) break;
    }
    return sumlx / suml2;
}

}  // namespace

// One thread per 256-element superblock.
__global__ __launch_bounds__(64) void quantize_q4k_weights_kernel(const float* __restrict__ x, size_t nblocks,
                                                                  uint8_t* __restrict__ out) {
    const size_t ib = (size_t)blockIdx.x * 64 + threadIdx.x;
    if (ib >= nblocks) return;
    const float* xb = x + ib * QK_K;
    float scales[8], mins[8];
    for (int j = 0; j < 8; j++) {
        float v[32];
        load32(xb + 32 * j, v);
        make_qkx1_quants_15_5(v, scales[j], mins[j]);
    }
    float max_scale = 0.0f, max_min = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) max_scale = fmaxf(scales[j], max_scale);
#pragma unroll
    for (int j = 0; j < 8; j++) max_min = fmaxf(mins[j], max_min);
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint8_t sc[12] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int a = nearest_int(inv_scale * scales[j]);
        const int c = nearest_int(inv_min * mins[j]);
        const uint8_t ls = (uint8_t)(a < 63 ? a : 63);
        const uint8_t lm = (uint8_t)(c < 63 ? c : 63);
        if (j < 4) {
            sc[j] = ls;
            sc[j + 4] = lm;
        } else {
            sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sc[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    q4k_store(xb, sc, f32_to_f16_rne(max_scale / 63.0f), f32_to_f16_rne(max_min / 63.0f), out + ib * Q4K_BYTES);
}

// from_float_imatrix for Q4_K, one thread per superblock: sub-block j's
// element weights are imatrix[(ib % bpr) * 256 + 32 j + l] * sqrt(sigma2 +
// x^2), sigma2 = 2 * sum(x^2) / 256 over the superblock.
__global__ __launch_bounds__(64) void quantize_q4k_imatrix_kernel(const float* __restrict__ x, size_t nblocks,
                                                                  uint8_t* __restrict__ out,
                                                                  const float* __restrict__ imatrix, size_t bpr) {
    const size_t ib = (size_t)blockIdx.x * 64 + threadIdx.x;
    if (ib >= nblocks) return;
    const float* xb = x + ib * QK_K;
    const float* qb = imatrix + (ib % bpr) * QK_K;
    float sum_x2 = -0.0f;
    for (int j = 0; j < 8; j++) {
        float v[32];
        load32(xb + 32 * j, v);
#pragma unroll
        for (int i = 0; i < 32; i++) sum_x2 += v[i] * v[i];
    }
    const float sigma2 = 2.0f * sum_x2 / 256.0f;
    float scales[8], mins[8], sw[8];
    for (int j = 0; j < 8; j++) {
        float v[32], q[32], wt[32];
        load32(xb + 32 * j, v);
        load32(qb + 32 * j, q);
#pragma unroll
        for (int i = 0; i < 32; i++) wt[i] = q[i] * sqrtf(sigma2 + v[i] * v[i]);
        float sumw = -0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) sumw += wt[i];
        sw[j] = sumw;
        make_qkx3_quants_15(v, wt, scales[j], mins[j]);
    }
    int ls[8], lm[8];
    const float d_block = make_qp_quants_8(scales, ls, sw);
    const float m_block = make_qp_quants_8(mins, lm, sw);
    uint8_t sc[12] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = (uint8_t)ls[j];
            sc[j + 4] = (uint8_t)lm[j];
        } else {
            sc[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
    q4k_store(xb, sc, f32_to_f16_rne(d_block), f32_to_f16_rne(m_block), out + ib * Q4K_BYTES);
}

// One thread per superblock; the 256 codes L live in LDS (256 B per thread).
// With imatrix set (from_float_imatrix), superblock ib's groups are weighted by
// imatrix[(ib % bpr) * 256 ...] instead of x * x.
__global__ __launch_bounds__(64) void quantize_q6k_weights_kernel(const float* __restrict__ x, size_t nblocks,
                                                                  uint8_t* __restrict__ out,
                                                                  const float* __restrict__ imatrix, size_t bpr) {
    __shared__ int8_t Ls[64][QK_K];
    const size_t ib = (size_t)blockIdx.x * 64 + threadIdx.x;
    if (ib >= nblocks) return;
    int8_t* L = Ls[threadIdx.x];
    const float* xb = x + ib * QK_K;
    float scales[16];
    float max_scale = 0.0f, max_abs_scale = 0.0f;
    for (int g = 0; g < 16; g++) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = reinterpret_cast<const float4*>(xb + 16 * g)[i];
            v[4 * i] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
        int ls[16];
        const float s = make_qx_quants_16(v, ls, imatrix ? imatrix + (ib % bpr) * QK_K + 16 * g : nullptr);
#pragma unroll
        for (int i = 0; i < 16; i++) L[16 * g + i] = (int8_t)ls[i];
        scales[g] = s;
        const float as = fabsf(s);
        if (as > max_abs_scale) {
            max_abs_scale = as;
            max_scale = s;
        }
    }
    const float iscale = -128.0f / max_scale;
    const uint16_t dh = f32_to_f16_rne(1.0f / iscale);
    const float df = f16_to_f32(dh);
    int8_t sc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int v = nearest_int(iscale * scales[j]);
        sc[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < 16; j++) {
        const float d = df * (float)sc[j];
        if (d == 0.0f) continue;
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = reinterpret_cast<const float4*>(xb + 16 * j)[i];
            v[4 * i] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) L[16 * j + i] = (int8_t)(clampi(nearest_int(v[i] / d), -32, 31) + 32);
    }
    uint8_t* ob = out + ib * Q6K_BYTES;  // only 2-byte aligned: 16-bit stores
    for (int h = 0; h < 2; h++) {
        const int8_t* Lh = L + 128 * h;
        for (int l = 0; l < 32; l += 2) {
            uint8_t qlA[2], qlB[2], qhv[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int i = l + t;
                const uint8_t q1 = (uint8_t)(Lh[i] & 0xF), q2 = (uint8_t)(Lh[i + 32] & 0xF);
                const uint8_t q3 = (uint8_t)(Lh[i + 64] & 0xF), q4 = (uint8_t)(Lh[i + 96] & 0xF);
                qlA[t] = (uint8_t)(q1 | (q3 << 4));
                qlB[t] = (uint8_t)(q2 | (q4 << 4));
                qhv[t] = (uint8_t)((Lh[i] >> 4) | ((Lh[i + 32] >> 4) << 2) | ((Lh[i + 64] >> 4) << 4) |
                                   ((Lh[i + 96] >> 4) << 6));
            }
            *reinterpret_cast<uint16_t*>(ob + 64 * h + l) = (uint16_t)(qlA[0] | (qlA[1] << 8));
            *reinterpret_cast<uint16_t*>(ob + 64 * h + 32 + l) = (uint16_t)(qlB[0] | (qlB[1] << 8));
            *reinterpret_cast<uint16_t*>(ob + 128 + 32 * h + l) = (uint16_t)(qhv[0] | (qhv[1] << 8));
        }
    }
    for (int j = 0; j < 16; j += 2)
        *reinterpret_cast<uint16_t*>(ob + 192 + j) = (uint16_t)((uint8_t)sc[j] | ((uint8_t)sc[j + 1] << 8));
    *reinterpret_cast<uint16_t*>(ob + 208) = dh;
}

// Eight 32-element blocks per wavefront (the activation quantizer's arithmetic).
__global__ __launch_bounds__(64) void quantize_q8_0_weights_kernel(const float* __restrict__ x, size_t nblocks,
                                                                   uint8_t* __restrict__ out) {
    const int lane = threadIdx.x;
    const size_t blk = (size_t)blockIdx.x * 8 + (lane >> 3);
    const bool live = blk < nblocks;
    const Q80Wave r = q8_0_quantize_wave(x + blk * QK8_0, live, lane);
    if (!live) return;
    uint8_t* p = out + blk * Q8_0_BYTES;
    uint16_t* qs16 = reinterpret_cast<uint16_t*>(p + 2 + 4 * (lane & 7));
    qs16[0] = (uint16_t)(r.packed & 0xffffu);
    qs16[1] = (uint16_t)(r.packed >> 16);
    if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(p) = r.dbits;
}

hipError_t launch_quantize_weights(int dtype, const float* x, size_t nblocks, uint8_t* out, hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    switch (dtype) {
        case GGML_Q4K:
            hipLaunchKernelGGL(quantize_q4k_weights_kernel, dim3((unsigned)((nblocks + 63) / 64)), dim3(64), 0, s, x,
                               nblocks, out);
            break;
        case GGML_Q6K:
            hipLaunchKernelGGL(quantize_q6k_weights_kernel, dim3((unsigned)((nblocks + 63) / 64)), dim3(64), 0, s, x,
                               nblocks, out, nullptr, (size_t)1);
            break;
        case GGML_Q8_0:
            hipLaunchKernelGGL(quantize_q8_0_weights_kernel, dim3((unsigned)((nblocks + 7) / 8)), dim3(64), 0, s, x,
                               nblocks, out);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_quantize_weights_imatrix(int dtype, const float* x, size_t nblocks, const float* imatrix,
                                           size_t blocks_per_row, uint8_t* out, hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    if (blocks_per_row == 0 || !imatrix) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((nblocks + 63) / 64));
    switch (dtype) {
        case GGML_Q4K:
            hipLaunchKernelGGL(quantize_q4k_imatrix_kernel, grid, dim3(64), 0, s, x, nblocks, out, imatrix,
                               blocks_per_row);
            break;
        case GGML_Q6K:
            hipLaunchKernelGGL(quantize_q6k_weights_kernel, grid, dim3(64), 0, s, x, nblocks, out, imatrix,
                               blocks_per_row);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- synthetic inputs ----

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; r++) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint32_t hi0 = __umulhi(0xD2511F53u, c.x), lo0 = 0xD2511F53u * c.x;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c.z), lo1 = 0xCD9E8D57u * c.z;
        c = uint4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    }
    return c;
}

// Element i = lane i%4 of the Philox block at counter [i/4 lo, i/4 hi, base, stream].
__global__ void random_bits_kernel(uint32_t* __restrict__ y, size_t n, unsigned long long start,
                                   unsigned long long seed, uint32_t base, uint32_t stream) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const unsigned long long gi = start + i;
    const unsigned long long blk = gi / 4;
    const uint4 w = philox4x32_10(uint4{(uint32_t)blk, (uint32_t)(blk >> 32), base, stream}, (uint32_t)seed,
                                  (uint32_t)(seed >> 32));
    const uint32_t v[4] = {w.x, w.y, w.z, w.w};
    y[i] = v[gi % 4];
}

// N(mean, std): Philox block b gives two Box-Muller pairs (words 0,1 and 2,3)
// for elements 4b..4b+3, cos for even and sin for odd elements; computed in
// double.  The transcendental calls round differently from the host libm, so
// values agree with the CPU generator to ~1 ulp of f32, not bit for bit.
__global__ void normal_kernel(float* __restrict__ y, size_t n, unsigned long long seed, uint32_t stream, float mean,
                              float stdv) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (4 * b >= n) return;
    const uint4 w = philox4x32_10(uint4{(uint32_t)b, (uint32_t)((unsigned long long)b >> 32), 0u, stream},
                                  (uint32_t)seed, (uint32_t)(seed >> 32));
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const double u1 = ((double)(ws[2 * p] >> 8) + 1.0) * (1.0 / 16777216.0);
        const double u2 = (double)(ws[2 * p + 1] >> 8) * (1.0 / 16777216.0);
        const double r = sqrt(-2.0 * log(u1));
        const double th = 6.283185307179586476925286766559 * u2;
        const size_t i0 = 4 * b + 2 * p;
        if (i0 < n) y[i0] = (float)((double)mean + (double)stdv * (r * cos(th)));
        if (i0 + 1 < n) y[i0 + 1] = (float)((double)mean + (double)stdv * (r * sin(th)));
    }
}

hipError_t launch_random_bits(uint32_t* y, size_t n, unsigned long long start, unsigned long long seed, uint32_t base,
                              uint32_t stream, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(random_bits_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, n, start, seed, base,
                       stream);
    return hipGetLastError();
}

hipError_t launch_normal(float* y, size_t n, unsigned long long seed, uint32_t stream, float mean, float stdv,
                         hipStream_t s) {
    if (!n) return hipSuccess;
    const size_t blocks = (n + 3) / 4;
    hipLaunchKernelGGL(normal_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s, y, n, seed, stream, mean,
                       stdv);
    return hipGetLastError();
}

}  // namespace frq
