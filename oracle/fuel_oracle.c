/*
 * fuel_oracle.c -- CPU restatement of fuel's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the CPU baseline).  The product
 * library under fuel_amd/ never includes, links or calls this file.
 *
 * Build: see oracle/Makefile.  It MUST be compiled with -ffp-contract=off and
 * without fast-math: Rust never fuses a*b+c into an FMA unless the source
 * calls mul_add / an FMA intrinsic, so the restatement may not either.  The
 * AVX2 functions use explicit _mm256_fmadd_ps exactly where avx.rs does.
 *
 * Rust semantics restated here:
 *   - f32::round is half-away-from-zero (C roundf).
 *   - float -> int `as` casts saturate and map NaN to 0 (sat_i32 / sat_i8).
 *   - int -> int `as` casts truncate (plain C casts).
 *   - f32::max / f32::min ignore a NaN operand (C fmaxf / fminf).
 *   - Iterator::sum over f32 folds left starting from -0.0.
 */
#include "fuel_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__x86_64__)
#include <immintrin.h>
#define FO_X86 1
#endif

_Static_assert(sizeof(fo_block_q8_0) == 34, "BlockQ8_0 is 34 bytes");
_Static_assert(sizeof(fo_block_q4k) == 144, "BlockQ4K is 144 bytes");
_Static_assert(sizeof(fo_block_q6k) == 210, "BlockQ6K is 210 bytes");
_Static_assert(sizeof(fo_block_q8k) == 292, "BlockQ8K is 292 bytes");

/* ------------------------------------------------------------------ */
/* Rust cast helpers                                                    */
/* ------------------------------------------------------------------ */

/* `f as i32` (saturating, NaN -> 0). */
static inline int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

/* `f as i8` (saturating, NaN -> 0). */
static inline int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* utils.rs:1-3 nearest_int: v.round() as i32 */
static inline int32_t nearest_int(float v) { return sat_i32(roundf(v)); }

static inline int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* f32::total_cmp: compare the sign-magnitude bit patterns as a total order. */
static inline int32_t total_key(float f) {
    int32_t b;
    memcpy(&b, &f, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

size_t fo_type_size(int t) {
    switch (t) {
    case FO_Q8_0: return 34;
    case FO_Q4K: return 144;
    case FO_Q6K: return 210;
    case FO_Q8K: return 292;
    default: return 0;
    }
}

size_t fo_block_size(int t) {
    switch (t) {
    case FO_Q8_0: return 32;
    case FO_Q4K:
    case FO_Q6K:
    case FO_Q8K: return 256;
    default: return 0;
    }
}

/* ------------------------------------------------------------------ */
/* f16 <-> f32 (half 2.5: IEEE binary16, round-to-nearest-even)         */
/* ------------------------------------------------------------------ */

float fo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
        if (man) bits |= 0x00400000u; /* quiet NaN */
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: value = man * 2^-24, exact in f32 */
            float v = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t fo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {
        if (man == 0) return sign | 0x7c00u;
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00u; /* overflow -> inf */
    if (e <= 0) {
        /* result is subnormal or zero: shift the full significand */
        if (e < -10) return sign; /* below half of the smallest subnormal */
        uint32_t sig = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e); /* 14..24 */
        uint32_t q = sig >> shift;
        uint32_t rem = sig & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry into inf */
    return (uint16_t)(sign | q);
}

/* bulk helpers for exhaustive checks */
void fo_f32_to_f16_array(const float *x, size_t n, uint16_t *y) {
    for (size_t i = 0; i < n; i++) y[i] = fo_f32_to_f16(x[i]);
}
void fo_f16_to_f32_array(const uint16_t *x, size_t n, float *y) {
    for (size_t i = 0; i < n; i++) y[i] = fo_f16_to_f32(x[i]);
}
/* F16C hardware conversion (vcvtps2ph, RNE) for cross-checking; returns
 * -1 when the host lacks F16C. */
#if FO_X86
__attribute__((target("f16c"))) static void f16c_convert(const float *x, size_t n, uint16_t *y) {
    for (size_t i = 0; i < n; i++) {
        __m128 v = _mm_set_ss(x[i]);
        __m128i h = _mm_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT);
        y[i] = (uint16_t)_mm_extract_epi16(h, 0);
    }
}
#endif
int fo_f32_to_f16_f16c(const float *x, size_t n, uint16_t *y) {
#if FO_X86
    if (!__builtin_cpu_supports("f16c")) return -1;
    f16c_convert(x, n, y);
    return 0;
#else
    (void)x; (void)n; (void)y;
    return -1;
#endif
}

/* ------------------------------------------------------------------ */
/* Philox-4x32-10 (fuel-cpu-kernels/src/philox.rs:13-135)               */
/* ------------------------------------------------------------------ */

void fo_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; r++) {
        if (r > 0) { /* rounds 2..10 bump the key first (philox.rs:57-67) */
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* random_bits_fill (philox.rs:120-133): element i is lane i%4 of the Philox
 * block at counter [block_lo, block_hi, base, stream], block = i/4, key = seed. */
void fo_random_bits_fill(uint32_t *dst, size_t n, uint64_t start, uint64_t seed, uint32_t base,
                         uint32_t stream) {
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    size_t i = 0;
    while (i < n) {
        uint64_t gi = start + i;
        uint64_t blk = gi / 4;
        uint32_t lane = (uint32_t)(gi % 4);
        uint32_t ctr[4] = {(uint32_t)blk, (uint32_t)(blk >> 32), base, stream};
        uint32_t w[4];
        fo_philox4x32_10(ctr, key, w);
        for (uint32_t l = lane; l < 4 && i < n; l++) dst[i++] = w[l];
    }
}

void fo_normal_fill(float *dst, size_t n, uint64_t seed, uint32_t stream, float mean, float std) {
    const double two_pi = 6.283185307179586476925286766559;
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
#pragma omp parallel for schedule(static)
    for (size_t b = 0; b < (n + 3) / 4; b++) {
        uint32_t ctr[4] = {(uint32_t)b, (uint32_t)((uint64_t)b >> 32), 0u, stream};
        uint32_t w[4];
        fo_philox4x32_10(ctr, key, w);
        for (int p = 0; p < 2; p++) {
            double u1 = ((double)(w[2 * p] >> 8) + 1.0) * (1.0 / 16777216.0);
            double u2 = (double)(w[2 * p + 1] >> 8) * (1.0 / 16777216.0);
            double r = sqrt(-2.0 * log(u1));
            double th = two_pi * u2;
            size_t i0 = 4 * b + 2 * p;
            if (i0 < n) dst[i0] = (float)((double)mean + (double)std * (r * cos(th)));
            if (i0 + 1 < n) dst[i0 + 1] = (float)((double)mean + (double)std * (r * sin(th)));
        }
    }
}

void fo_uniform_u32_fill(uint32_t *dst, size_t n, uint64_t seed, uint32_t stream, uint32_t bound) {
    fo_random_bits_fill(dst, n, 0, seed, 0, stream);
    for (size_t i = 0; i < n; i++) dst[i] = (uint32_t)(((uint64_t)dst[i] * bound) >> 32);
}

/* ------------------------------------------------------------------ */
/* Activation quantizers                                                */
/* ------------------------------------------------------------------ */

/* BlockQ8K::from_float (k_quants.rs:2230-2267). */
void fo_quantize_q8k(const float *x, size_t k, fo_block_q8k *y) {
    size_t nb = k / FO_QK_K;
    for (size_t i = 0; i < nb; i++) {
        const float *xs = x + i * FO_QK_K;
        fo_block_q8k *b = &y[i];
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < FO_QK_K; j++) {
            float ax = fabsf(xs[j]);
            if (amax < ax) { /* strict: the first element of largest |x| wins */
                amax = ax;
                max = xs[j];
            }
        }
        if (amax == 0.0f) {
            /* matmul hands a zero-initialised buffer (k_quants.rs:2304), so
             * bsums stay 0 on this branch. */
            b->d = 0.0f;
            memset(b->qs, 0, sizeof b->qs);
            memset(b->bsums, 0, sizeof b->bsums);
            continue;
        }
        float iscale = -128.0f / max;
        for (int j = 0; j < FO_QK_K; j++) {
            float v = roundf(iscale * xs[j]);
            b->qs[j] = sat_i8(fminf(v, 127.0f));
        }
        for (int g = 0; g < 16; g++) {
            int32_t s = 0;
            for (int l = 0; l < 16; l++) s += b->qs[16 * g + l];
            b->bsums[g] = (int16_t)s;
        }
        b->d = 1.0f / iscale;
    }
}

/* BlockQ8_0::from_float (k_quants.rs:629-658). */
void fo_quantize_q8_0(const float *x, size_t k, fo_block_q8_0 *y) {
    size_t nb = k / FO_QK8_0;
    for (size_t i = 0; i < nb; i++) {
        const float *xs = x + i * FO_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < FO_QK8_0; j++) amax = fmaxf(amax, fabsf(xs[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = fo_f32_to_f16(d);
        for (int j = 0; j < FO_QK8_0; j++) y[i].qs[j] = sat_i8(roundf(xs[j] * id));
    }
}

/* ------------------------------------------------------------------ */
/* Weight quantizers                                                    */
/* ------------------------------------------------------------------ */

/* utils.rs:50-60 get_scale_min_k4 */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* utils.rs:229-286 make_qkx1_quants(nmax, ntry, x): returns (scale, -min). */
static void make_qkx1_quants(int nmax, int ntry, const float *x, int n, float *out_scale,
                             float *out_min) {
    uint8_t l[64];
    memset(l, 0, sizeof l);
    float mn = x[0], mx = x[0];
    int32_t kmn = total_key(x[0]), kmx = kmn;
    for (int i = 1; i < n; i++) {
        int32_t kk = total_key(x[i]);
        if (kk < kmn) { kmn = kk; mn = x[i]; } /* min_by keeps the first minimum */
        if (kk >= kmx) { kmx = kk; mx = x[i]; } /* max_by keeps the last maximum */
    }
    if (mx == mn) {
        *out_scale = 0.0f;
        *out_min = 0.0f;
        return;
    }
    float min = fminf(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int t = 0; t < ntry; t++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        for (int i = 0; i < n; i++) {
            int32_t li = clamp_i32(nearest_int(iscale * (x[i] - min)), 0, nmax);
            uint8_t cl = (uint8_t)li;
            if (cl != l[i]) {
                l[i] = cl;
                did_change = 1;
            }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
        for (int i = 0; i < n; i++) sum += x[i] - scale * (float)l[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *out_scale = scale;
    *out_min = -min;
}

/* The 4-bit codes of a Q4_K superblock from its d, dmin and packed scales
 * (k_quants.rs:1511-1527, also the tail of from_float_imatrix). */
static void q4k_codes(const float *x, fo_block_q4k *b) {
    uint8_t L[FO_QK_K];
    memset(L, 0, sizeof L);
    for (int j = 0; j < 8; j++) {
        uint8_t sc, m;
        get_scale_min_k4(j, b->scales, &sc, &m);
        float d = fo_f16_to_f32(b->d) * (float)sc;
        if (d != 0.0f) {
            float dm = fo_f16_to_f32(b->dmin) * (float)m;
            for (int ii = 0; ii < 32; ii++) {
                int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);
                L[32 * j + ii] = (uint8_t)clamp_i32(lv, 0, 15);
            }
        }
    }
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) b->qs[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + l + 32] << 4));
}

/* BlockQ4K::from_float (k_quants.rs:1470-1528). */
void fo_quantize_q4k(const float *xin, size_t k, fo_block_q4k *y) {
    size_t nb = k / FO_QK_K;
    for (size_t ib = 0; ib < nb; ib++) {
        const float *x = xin + ib * FO_QK_K;
        fo_block_q4k *b = &y[ib];
        memset(b, 0, sizeof *b);
        float scales[8], mins[8];
        for (int j = 0; j < 8; j++) make_qkx1_quants(15, 5, x + 32 * j, 32, &scales[j], &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) max_scale = fmaxf(scales[j], max_scale);
        for (int j = 0; j < 8; j++) max_min = fmaxf(mins[j], max_min);
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        for (int j = 0; j < 8; j++) {
            int32_t a = nearest_int(inv_scale * scales[j]);
            int32_t c = nearest_int(inv_min * mins[j]);
            uint8_t ls = (uint8_t)(a < 63 ? a : 63);
            uint8_t lm = (uint8_t)(c < 63 ? c : 63);
            if (j < 4) {
                b->scales[j] = ls;
                b->scales[j + 4] = lm;
            } else {
                b->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                b->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                b->scales[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        b->d = fo_f32_to_f16(max_scale / 63.0f);
        b->dmin = fo_f32_to_f16(max_min / 63.0f);
        q4k_codes(x, b);
    }
}

/* utils.rs:358-469 make_qkx3_quants(nmax, x, Some(weights), rmin, rdelta,
 * nstep, use_mad = false): returns (scale, -min). */
static void make_qkx3_quants_w(int nmax, const float *x, const float *w, int n, float rmin, float rdelta, int nstep,
                               float *out_scale, float *out_neg_min) {
    uint8_t l[32], laux[32];
    float min_val = x[0], max_val = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < min_val) min_val = x[i];
        if (x[i] > max_val) max_val = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (min_val > 0.0f) min_val = 0.0f;
    if (max_val <= min_val) {
        *out_scale = 0.0f;
        *out_neg_min = -min_val;
        return;
    }
    float iscale = (float)nmax / (max_val - min_val);
    float scale = 1.0f / iscale;
    float best_mad = 0.0f;
    for (int i = 0; i < n; i++) {
        uint8_t lv = (uint8_t)clamp_i32(nearest_int(iscale * (x[i] - min_val)), 0, nmax);
        l[i] = lv;
        float diff = scale * (float)lv + min_val - x[i];
        diff = diff * diff;
        best_mad += w[i] * diff;
    }
    if (nstep >= 1) {
        for (int is = 0; is <= nstep; is++) {
            iscale = (rmin + rdelta * (float)is + (float)nmax) / (max_val - min_val);
            float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
            for (int i = 0; i < n; i++) {
                uint8_t lv = (uint8_t)clamp_i32(nearest_int(iscale * (x[i] - min_val)), 0, nmax);
                laux[i] = lv;
                sum_l += w[i] * (float)lv;
                sum_l2 += w[i] * ((float)lv * (float)lv);
                sum_xl += w[i] * (float)lv * x[i];
            }
            float d = sum_w * sum_l2 - sum_l * sum_l;
            if (d > 0.0f) {
                float this_scale = (sum_w * sum_xl - sum_x * sum_l) / d;
                float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / d;
                if (this_min > 0.0f) {
                    this_min = 0.0f;
                    this_scale = sum_xl / sum_l2;
                }
                float mad = 0.0f;
                for (int i = 0; i < n; i++) {
                    float diff = this_scale * (float)laux[i] + this_min - x[i];
                    diff = diff * diff;
                    mad += w[i] * diff;
                }
                if (mad < best_mad) {
                    memcpy(l, laux, sizeof l);
                    best_mad = mad;
                    scale = this_scale;
                    min_val = this_min;
                }
            }
        }
    }
    *out_scale = scale;
    *out_neg_min = -min_val;
}

/* Rust `f as u8` for a float: saturating, NaN -> 0. */
static inline uint8_t sat_u8(float v) {
    if (v != v || v <= 0.0f) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}

/* utils.rs:472-563 make_qp_quants(n, nmax, x, l, quant_weights): the scale
 * of n non-negative values on 0..nmax by a grid search over iscale and a
 * coordinate descent, weighted; returns sumlx / suml2. */
static float make_qp_quants(int n, int nmax, const float *x, uint8_t *l, const float *qw) {
    float max = 0.0f;
    for (int i = 0; i < n; i++) max = fmaxf(max, x[i]); /* f32::max: a NaN operand is ignored */
    if (max == 0.0f) {
        for (int i = 0; i < n; i++) l[i] = 0;
        return 0.0f;
    }
    float iscale = (float)nmax / max;
    for (int i = 0; i < n; i++) l[i] = (uint8_t)nearest_int(iscale * x[i]); /* i32 as u8: wraps */
    float scale = 1.0f / iscale;
    float best_mse = -0.0f;
    for (int i = 0; i < n; i++) {
        float diff = x[i] - scale * (float)l[i];
        best_mse += qw[i] * diff * diff;
    }
    for (int is = -4; is <= 4; is++) {
        if (is == 0) continue;
        float iscale_is = (0.1f * (float)is + (float)nmax) / max;
        float scale_is = 1.0f / iscale_is;
        float mse = -0.0f;
        for (int i = 0; i < n; i++) {
            uint8_t li = (uint8_t)nearest_int(iscale_is * x[i]);
            if (li > nmax) li = (uint8_t)nmax;
            float diff = x[i] - scale_is * (float)li;
            mse += qw[i] * diff * diff;
        }
        if (mse < best_mse) {
            best_mse = mse;
            iscale = iscale_is;
        }
    }
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        uint8_t li = sat_u8(roundf(iscale * x[i]));
        if (li > nmax) li = (uint8_t)nmax;
        l[i] = li;
        sumlx += qw[i] * x[i] * (float)li;
        suml2 += qw[i] * ((float)li * (float)li);
    }
    for (int it = 0; it < 5; it++) {
        int n_changed = 0;
        for (int i = 0; i < n; i++) {
            float slx = sumlx - qw[i] * x[i] * (float)l[i];
            float sl2 = suml2 - qw[i] * ((float)l[i] * (float)l[i]);
            if (slx > 0.0f && sl2 > 0.0f) {
                uint8_t new_li = (uint8_t)nearest_int(x[i] * sl2 / slx);
                if (new_li > nmax) new_li = (uint8_t)nmax;
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

/* BlockQ4K::from_float_imatrix (k_quants.rs:1530-1593), one superblock; qw =
 * the superblock's 256 importance weights. */
static void q4k_block_imatrix(const float *x, const float *qw, fo_block_q4k *b) {
    memset(b, 0, sizeof *b);
    float mins[8], scales[8], weights[32], sw[8];
    uint8_t ls[8], lm[8];
    float sum_x2 = -0.0f;
    for (int i = 0; i < FO_QK_K; i++) sum_x2 += x[i] * x[i];
    float sigma2 = 2.0f * sum_x2 / (float)FO_QK_K;
    for (int j = 0; j < 8; j++) {
        for (int l = 0; l < 32; l++) {
            float xe = x[32 * j + l];
            weights[l] = qw[32 * j + l] * sqrtf(sigma2 + xe * xe);
        }
        float sumw = -0.0f;
        for (int l = 0; l < 32; l++) sumw += weights[l];
        sw[j] = sumw;
        make_qkx3_quants_w(15, x + 32 * j, weights, 32, -0.9f, 0.05f, 36, &scales[j], &mins[j]);
    }
    float d_block = make_qp_quants(8, 63, scales, ls, sw);
    float m_block = make_qp_quants(8, 63, mins, lm, sw);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            b->scales[j] = ls[j];
            b->scales[j + 4] = lm[j];
        } else {
            b->scales[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            b->scales[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            b->scales[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
    b->d = fo_f32_to_f16(d_block);
    b->dmin = fo_f32_to_f16(m_block);
    q4k_codes(x, b);
}

static void q6k_block(const float *x, const float *qw, int8_t *L, fo_block_q6k *b);

/* from_float_imatrix over a tensor of k elements (whole superblocks): the
 * superblock with flat index s takes the importance weights of column block
 * s % (n_per_row / 256) (k_quants.rs:1544, 2092).  Q4_K and Q6_K only. */
int fo_quantize_imatrix(int t, const float *x, size_t k, const float *imatrix, size_t n_per_row, void *y) {
    if (n_per_row < FO_QK_K || n_per_row % FO_QK_K || k % FO_QK_K) return -1;
    size_t nbr = n_per_row / FO_QK_K;
    if (t == FO_Q4K) {
        for (size_t s = 0; s < k / FO_QK_K; s++)
            q4k_block_imatrix(x + s * FO_QK_K, imatrix + (s % nbr) * FO_QK_K, (fo_block_q4k *)y + s);
        return 0;
    }
    if (t == FO_Q6K) {
        int8_t L[FO_QK_K];
        memset(L, 0, sizeof L);
        for (size_t s = 0; s < k / FO_QK_K; s++)
            q6k_block(x + s * FO_QK_K, imatrix + (s % nbr) * FO_QK_K, L, (fo_block_q6k *)y + s);
        return 0;
    }
    return -1;
}

/* utils.rs:62-226 make_qx_quants with rmse_type = 1, as BlockQ6K::from_float
 * (qw = null: weights w = x*x) and from_float_imatrix (qw = the importance
 * weights) call it. */
static float make_qx_quants_w(int n, int nmax, const float *x, int8_t *ls, const float *qw) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax == 0.0f) {
        for (int i = 0; i < n; i++) ls[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        int32_t l = clamp_i32(nearest_int(iscale * x[i]), -nmax, nmax - 1);
        ls[i] = (int8_t)(l + nmax);
        float w = qw ? qw[i] : x[i] * x[i];
        float lf = (float)l;
        sumlx += w * x[i] * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        float is2 = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        int changed = 0;
        for (int i = 0; i < n; i++) {
            int32_t l = clamp_i32(nearest_int(is2 * x[i]), -nmax, nmax - 1);
            if (l + nmax != (int32_t)ls[i]) changed = 1;
            float w = qw ? qw[i] : x[i] * x[i];
            float lf = (float)l;
            slx += w * x[i] * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
        for (int i = 0; i < n; i++) {
            int32_t l = nearest_int(is2 * x[i]);
            ls[i] = (int8_t)(nmax + clamp_i32(l, -nmax, nmax - 1));
        }
        sumlx = slx;
        suml2 = sl2;
        scale = sumlx / suml2;
        best = scale * sumlx;
    }
    for (int itry = 0; itry < 5; itry++) {
        int n_changed = 0;
        for (int i = 0; i < n; i++) {
            float w = qw ? qw[i] : x[i] * x[i];
            int32_t l = (int32_t)ls[i] - nmax;
            float slx = sumlx - w * x[i] * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                int32_t new_l = clamp_i32(nearest_int(x[i] * sl2 / slx), -nmax, nmax - 1);
                if (new_l != l) {
                    slx += w * x[i] * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        ls[i] = (int8_t)(nmax + new_l);
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
    (void)best;
    return scale;
}

/* One superblock of BlockQ6K::from_float (qw = NULL) or of
 * from_float_imatrix (k_quants.rs:2077-2145: qw = the superblock's 256
 * importance weights).  L carries the codes from block to block, as the
 * reference's buffer does. */
static void q6k_block(const float *x, const float *qw, int8_t *L, fo_block_q6k *b) {
    {
        memset(b, 0, sizeof *b);
        float scales[16];
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int ib = 0; ib < 16; ib++) {
            float s = make_qx_quants_w(16, 32, x + 16 * ib, L + 16 * ib, qw ? qw + 16 * ib : NULL);
            scales[ib] = s;
            float as = fabsf(s);
            if (as > max_abs_scale) {
                max_abs_scale = as;
                max_scale = s;
            }
        }
        float iscale = -128.0f / max_scale;
        b->d = fo_f32_to_f16(1.0f / iscale);
        for (int j = 0; j < 16; j++) {
            int32_t v = nearest_int(iscale * scales[j]);
            b->scales[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            float d = fo_f16_to_f32(b->d) * (float)b->scales[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ii++) {
                int32_t ll = clamp_i32(nearest_int(x[16 * j + ii] / d), -32, 31);
                L[16 * j + ii] = (int8_t)(ll + 32);
            }
        }
        for (int h = 0; h < 2; h++) {
            const int8_t *Lh = L + 128 * h;
            uint8_t *ql = b->ql + 64 * h;
            uint8_t *qh = b->qh + 32 * h;
            for (int l = 0; l < 32; l++) {
                uint8_t q1 = (uint8_t)(Lh[l] & 0xF), q2 = (uint8_t)(Lh[l + 32] & 0xF);
                uint8_t q3 = (uint8_t)(Lh[l + 64] & 0xF), q4 = (uint8_t)(Lh[l + 96] & 0xF);
                ql[l] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) |
                                  ((Lh[l + 96] >> 4) << 6));
            }
        }
    }
}

/* BlockQ6K::from_float (k_quants.rs:2005-2075). */
void fo_quantize_q6k(const float *xin, size_t k, fo_block_q6k *y) {
    int8_t L[FO_QK_K];
    memset(L, 0, sizeof L);
    for (size_t ibk = 0; ibk < k / FO_QK_K; ibk++) q6k_block(xin + ibk * FO_QK_K, NULL, L, &y[ibk]);
}

void fo_quantize_rows(int t, const float *x, size_t rows, size_t k, void *y) {
    size_t bpr = k / fo_block_size(t);
    size_t ts = fo_type_size(t);
#pragma omp parallel for schedule(dynamic, 16)
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * k;
        void *yr = (char *)y + r * bpr * ts;
        switch (t) {
        case FO_Q8_0: fo_quantize_q8_0(xr, k, (fo_block_q8_0 *)yr); break;
        case FO_Q4K: fo_quantize_q4k(xr, k, (fo_block_q4k *)yr); break;
        case FO_Q6K: fo_quantize_q6k(xr, k, (fo_block_q6k *)yr); break;
        case FO_Q8K: fo_quantize_q8k(xr, k, (fo_block_q8k *)yr); break;
        default: break;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Dequantizers (to_float)                                              */
/* ------------------------------------------------------------------ */

/* k_quants.rs:1595-1622 */
static void dequant_q4k(const fo_block_q4k *xs, size_t k, float *y) {
    for (size_t ib = 0; ib < k / FO_QK_K; ib++) {
        const fo_block_q4k *b = &xs[ib];
        float d = fo_f16_to_f32(b->d), mn = fo_f16_to_f32(b->dmin);
        float *yy = y + ib * FO_QK_K;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            get_scale_min_k4(2 * c, b->scales, &sc, &m);
            float d1 = d * (float)sc, m1 = mn * (float)m;
            get_scale_min_k4(2 * c + 1, b->scales, &sc, &m);
            float d2 = d * (float)sc, m2 = mn * (float)m;
            const uint8_t *q = b->qs + 32 * c;
            for (int l = 0; l < 32; l++) yy[64 * c + l] = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) yy[64 * c + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
        }
    }
}

/* k_quants.rs:2158-2189 */
static void dequant_q6k(const fo_block_q6k *xs, size_t k, float *y) {
    for (size_t ib = 0; ib < k / FO_QK_K; ib++) {
        const fo_block_q6k *b = &xs[ib];
        float d = fo_f16_to_f32(b->d);
        for (int h = 0; h < 2; h++) {
            float *yy = y + ib * FO_QK_K + 128 * h;
            const int8_t *sc = b->scales + 8 * h;
            const uint8_t *ql = b->ql + 64 * h;
            const uint8_t *qh = b->qh + 32 * h;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int8_t q1 = (int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int8_t q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                yy[l] = d * (float)sc[is] * (float)q1;
                yy[l + 32] = d * (float)sc[is + 2] * (float)q2;
                yy[l + 64] = d * (float)sc[is + 4] * (float)q3;
                yy[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

void fo_dequantize(int t, const void *blocks, size_t k, float *y) {
    switch (t) {
    case FO_Q8_0: { /* k_quants.rs:611-627 */
        const fo_block_q8_0 *b = (const fo_block_q8_0 *)blocks;
        for (size_t i = 0; i < k / 32; i++) {
            float d = fo_f16_to_f32(b[i].d);
            for (int j = 0; j < 32; j++) y[32 * i + j] = (float)b[i].qs[j] * d;
        }
        break;
    }
    case FO_Q4K: dequant_q4k((const fo_block_q4k *)blocks, k, y); break;
    case FO_Q6K: dequant_q6k((const fo_block_q6k *)blocks, k, y); break;
    case FO_Q8K: { /* k_quants.rs:2269-2280 */
        const fo_block_q8k *b = (const fo_block_q8k *)blocks;
        for (size_t i = 0; i < k / 256; i++)
            for (int j = 0; j < 256; j++) y[256 * i + j] = b[i].d * (float)b[i].qs[j];
        break;
    }
    default: break;
    }
}

/* ------------------------------------------------------------------ */
/* Scalar vec_dot_unopt                                                 */
/* ------------------------------------------------------------------ */

/* The utmp unpack of k_quants.rs:1427-1437 (12 packed bytes -> 8 scales
 * and 8 mins).  Kept as its own routine so a test can check it against
 * get_scale_min_k4 over random bytes. */
void fo_q4k_unpack_scales(const uint8_t packed[12], uint8_t scales[8], uint8_t mins[8]) {
    uint32_t u0, u1, u2;
    memcpy(&u0, packed, 4);
    memcpy(&u1, packed + 4, 4);
    memcpy(&u2, packed + 8, 4);
    uint32_t u3 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
    uint32_t t = u1 & 0x3f3f3f3fu;
    u1 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
    u2 = t;
    u0 &= 0x3f3f3f3fu;
    memcpy(scales, &u0, 4);
    memcpy(scales + 4, &u1, 4);
    memcpy(mins, &u2, 4);
    memcpy(mins + 4, &u3, 4);
}

/* k_quants.rs:1388-1468 */
float fo_vec_dot_q4k_unopt(size_t k, const fo_block_q4k *xs, const fo_block_q8k *ys) {
    float sums[8] = {0};
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / FO_QK_K; ib++) {
        const fo_block_q4k *x = &xs[ib];
        const fo_block_q8k *y = &ys[ib];
        int8_t a[FO_QK_K];
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                a[64 * c + l] = (int8_t)(x->qs[32 * c + l] & 0xF);
                a[64 * c + 32 + l] = (int8_t)(x->qs[32 * c + l] >> 4);
            }
        uint8_t scales[8], mins[8];
        fo_q4k_unpack_scales(x->scales, scales, mins);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
        int32_t aux32[8] = {0};
        for (int s = 0; s < 8; s++)
            for (int g = 0; g < 4; g++)
                for (int l = 0; l < 8; l++) {
                    int idx = 32 * s + 8 * g + l;
                    int16_t p = (int16_t)(y->qs[idx] * a[idx]);
                    aux32[l] += (int32_t)scales[s] * (int32_t)p;
                }
        float d = fo_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = fo_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}

static inline void q6k_unpack(const fo_block_q6k *x, int8_t a[FO_QK_K]) {
    for (int h = 0; h < 2; h++) {
        const uint8_t *q4 = x->ql + 64 * h;
        const uint8_t *qh = x->qh + 32 * h;
        int8_t *aa = a + 128 * h;
        for (int l = 0; l < 32; l++) {
            aa[l] = (int8_t)((int32_t)((q4[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
            aa[l + 32] = (int8_t)((int32_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
            aa[l + 64] = (int8_t)((int32_t)((q4[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
            aa[l + 96] = (int8_t)((int32_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
        }
    }
}

/* k_quants.rs:1946-2003 */
float fo_vec_dot_q6k_unopt(size_t k, const fo_block_q6k *xs, const fo_block_q8k *ys) {
    float sums[8] = {0};
    for (size_t ib = 0; ib < k / FO_QK_K; ib++) {
        const fo_block_q6k *x = &xs[ib];
        const fo_block_q8k *y = &ys[ib];
        int8_t a[FO_QK_K];
        q6k_unpack(x, a);
        float aux32[8] = {0};
        for (int j = 0; j < 16; j++) {
            float scale = (float)x->scales[j];
            for (int half = 0; half < 2; half++)
                for (int l = 0; l < 8; l++) {
                    int idx = 16 * j + 8 * half + l;
                    int16_t p = (int16_t)(y->qs[idx] * a[idx]);
                    aux32[l] += scale * (float)p;
                }
        }
        float d = fo_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

/* k_quants.rs:674-692 */
float fo_vec_dot_q8_0_unopt(size_t k, const fo_block_q8_0 *xs, const fo_block_q8_0 *ys) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / FO_QK8_0; ib++) {
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)xs[ib].qs[j] * (int32_t)ys[ib].qs[j];
        sumf += (float)s * fo_f16_to_f32(xs[ib].d) * fo_f16_to_f32(ys[ib].d);
    }
    return sumf;
}

/* ------------------------------------------------------------------ */
/* Integer taps                                                         */
/* ------------------------------------------------------------------ */

void fo_block_isums(int t, size_t k, const void *w_row, const void *a_row, int32_t *isum,
                    int32_t *msum) {
    if (t == FO_Q4K) {
        const fo_block_q4k *w = (const fo_block_q4k *)w_row;
        const fo_block_q8k *a = (const fo_block_q8k *)a_row;
        for (size_t b = 0; b < k / FO_QK_K; b++) {
            uint8_t sc[8], mn[8];
            fo_q4k_unpack_scales(w[b].scales, sc, mn);
            int32_t s = 0, m = 0;
            for (int c = 0; c < 4; c++) {
                int32_t lo = 0, hi = 0;
                for (int l = 0; l < 32; l++) {
                    lo += (int32_t)(w[b].qs[32 * c + l] & 0xF) * a[b].qs[64 * c + l];
                    hi += (int32_t)(w[b].qs[32 * c + l] >> 4) * a[b].qs[64 * c + 32 + l];
                }
                s += (int32_t)sc[2 * c] * lo + (int32_t)sc[2 * c + 1] * hi;
            }
            for (int g = 0; g < 16; g++) m += (int32_t)a[b].bsums[g] * (int32_t)mn[g / 2];
            isum[b] = s;
            msum[b] = m;
        }
    } else if (t == FO_Q6K) {
        const fo_block_q6k *w = (const fo_block_q6k *)w_row;
        const fo_block_q8k *a = (const fo_block_q8k *)a_row;
        for (size_t b = 0; b < k / FO_QK_K; b++) {
            int8_t q[FO_QK_K];
            q6k_unpack(&w[b], q);
            int32_t s = 0;
            for (int g = 0; g < 16; g++) {
                int32_t p = 0;
                for (int l = 0; l < 16; l++) p += (int32_t)q[16 * g + l] * a[b].qs[16 * g + l];
                s += (int32_t)w[b].scales[g] * p;
            }
            isum[b] = s;
            msum[b] = 0;
        }
    } else if (t == FO_Q8_0) {
        const fo_block_q8_0 *w = (const fo_block_q8_0 *)w_row;
        const fo_block_q8_0 *a = (const fo_block_q8_0 *)a_row;
        for (size_t b = 0; b < k / FO_QK8_0; b++) {
            int32_t s = 0;
            for (int j = 0; j < 32; j++) s += (int32_t)w[b].qs[j] * a[b].qs[j];
            isum[b] = s;
            msum[b] = 0;
        }
    }
}

/* ------------------------------------------------------------------ */
/* AVX2 vec_dot (avx.rs)                                                */
/* ------------------------------------------------------------------ */

int fo_have_avx2(void) {
#if FO_X86
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
    return 0;
#endif
}

#if FO_X86
#define AVX2_FN __attribute__((target("avx2,fma")))

/* avx.rs:26-32 hsum_float_8: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) */
AVX2_FN static inline float hsum8(__m256 v) {
    __m128 r = _mm_add_ps(_mm256_extractf128_ps(v, 1), _mm256_castps256_ps128(v));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}

/* avx.rs:597-681 vec_dot_q4k_q8k.  i32 lane u of the per-superblock sum
 * collects the products of bytes 4u..4u+3 of every 32-byte quant vector,
 * each pair-summed then scaled by that vector's sub-block scale. */
AVX2_FN static float q4k_avx2(size_t k, const fo_block_q4k *xs, const fo_block_q8k *ys) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256 acc = _mm256_setzero_ps();
    __m128 acc_m = _mm_setzero_ps();
    for (size_t ib = 0; ib < k / FO_QK_K; ib++) {
        const fo_block_q4k *x = &xs[ib];
        const fo_block_q8k *y = &ys[ib];
        float d = y->d * fo_f16_to_f32(x->d);
        float dmin = -y->d * fo_f16_to_f32(x->dmin);
        uint8_t sc8[8], mn8[8];
        fo_q4k_unpack_scales(x->scales, sc8, mn8);
        /* mins as 8 x i16 against the pairwise-summed bsums: lane v gets
         * m[2v]*(b[4v]+b[4v+1]) + m[2v+1]*(b[4v+2]+b[4v+3]). */
        __m128i mins16 = _mm_cvtepu8_epi16(_mm_loadl_epi64((const __m128i *)mn8));
        __m128i bs_lo = _mm_loadu_si128((const __m128i *)y->bsums);
        __m128i bs_hi = _mm_loadu_si128((const __m128i *)(y->bsums + 8));
        __m128i pairs = _mm_hadd_epi16(bs_lo, bs_hi);
        __m128i prod = _mm_madd_epi16(mins16, pairs);
        acc_m = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), acc_m);

        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 4; c++) {
            __m256i sl = _mm256_set1_epi16((short)sc8[2 * c]);
            __m256i sh = _mm256_set1_epi16((short)sc8[2 * c + 1]);
            __m256i bits = _mm256_loadu_si256((const __m256i *)(x->qs + 32 * c));
            __m256i lo = _mm256_and_si256(bits, m4);
            __m256i hi = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
            __m256i ql8 = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * c));
            __m256i qh8 = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * c + 32));
            sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(sl, _mm256_maddubs_epi16(lo, ql8)));
            sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(sh, _mm256_maddubs_epi16(hi, qh8)));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    __m128 m = _mm_add_ps(acc_m, _mm_movehl_ps(acc_m, acc_m));
    m = _mm_add_ss(m, _mm_movehdup_ps(m));
    return hsum8(acc) + _mm_cvtss_f32(m);
}

/* avx.rs:285-372 vec_dot_q6k_q8k.  Unsigned 6-bit codes against q8, minus
 * 32*q8, pair-summed then multiplied by the 16-element group scale. */
AVX2_FN static float q6k_avx2(size_t k, const fo_block_q6k *xs, const fo_block_q8k *ys) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    const __m256i m2 = _mm256_set1_epi8(3);
    const __m256i k32 = _mm256_set1_epi8(32);
    __m256 acc = _mm256_setzero_ps();
    for (size_t ib = 0; ib < k / FO_QK_K; ib++) {
        const fo_block_q6k *x = &xs[ib];
        const fo_block_q8k *y = &ys[ib];
        float d = y->d * fo_f16_to_f32(x->d);
        __m256i sumi = _mm256_setzero_si256();
        for (int h = 0; h < 2; h++) {
            __m256i b1 = _mm256_loadu_si256((const __m256i *)(x->ql + 64 * h));
            __m256i b2 = _mm256_loadu_si256((const __m256i *)(x->ql + 64 * h + 32));
            __m256i bh = _mm256_loadu_si256((const __m256i *)(x->qh + 32 * h));
            __m256i q[4];
            q[0] = _mm256_or_si256(_mm256_and_si256(b1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(bh, m2), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(b2, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 2), m2), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 4), m2), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b2, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 6), m2), 4));
            for (int i = 0; i < 4; i++) {
                __m256i q8 = _mm256_loadu_si256((const __m256i *)(y->qs + 128 * h + 32 * i));
                __m256i p = _mm256_sub_epi16(_mm256_maddubs_epi16(q[i], q8), _mm256_maddubs_epi16(k32, q8));
                int g = 8 * h + 2 * i; /* 16-element groups g (bytes 0..15) and g+1 (16..31) */
                __m256i s = _mm256_setr_epi16(x->scales[g], x->scales[g], x->scales[g], x->scales[g],
                                              x->scales[g], x->scales[g], x->scales[g], x->scales[g],
                                              x->scales[g + 1], x->scales[g + 1], x->scales[g + 1],
                                              x->scales[g + 1], x->scales[g + 1], x->scales[g + 1],
                                              x->scales[g + 1], x->scales[g + 1]);
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(s, p));
            }
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum8(acc);
}

/* avx.rs:70-88 vec_dot_q8_0_q8_0 (with mul_sum_i8_pairs_float, avx.rs:13-48):
 * |x| * sign(y, x) through maddubs, pairs summed to i32 lanes of 4 products. */
AVX2_FN static float q8_0_avx2(size_t k, const fo_block_q8_0 *xs, const fo_block_q8_0 *ys) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (size_t ib = 0; ib < k / FO_QK8_0; ib++) {
        __m256 d = _mm256_set1_ps(fo_f16_to_f32(xs[ib].d) * fo_f16_to_f32(ys[ib].d));
        __m256i bx = _mm256_loadu_si256((const __m256i *)xs[ib].qs);
        __m256i by = _mm256_loadu_si256((const __m256i *)ys[ib].qs);
        __m256i ax = _mm256_sign_epi8(bx, bx);
        __m256i sy = _mm256_sign_epi8(by, bx);
        __m256 q = _mm256_cvtepi32_ps(_mm256_madd_epi16(ones, _mm256_maddubs_epi16(ax, sy)));
        acc = _mm256_fmadd_ps(d, q, acc);
    }
    return hsum8(acc);
}
#endif

float fo_vec_dot_q4k_avx2(size_t k, const fo_block_q4k *w, const fo_block_q8k *a) {
#if FO_X86
    if (fo_have_avx2()) return q4k_avx2(k, w, a);
#endif
    (void)k; (void)w; (void)a;
    return NAN;
}
float fo_vec_dot_q6k_avx2(size_t k, const fo_block_q6k *w, const fo_block_q8k *a) {
#if FO_X86
    if (fo_have_avx2()) return q6k_avx2(k, w, a);
#endif
    (void)k; (void)w; (void)a;
    return NAN;
}
float fo_vec_dot_q8_0_avx2(size_t k, const fo_block_q8_0 *w, const fo_block_q8_0 *a) {
#if FO_X86
    if (fo_have_avx2()) return q8_0_avx2(k, w, a);
#endif
    (void)k; (void)w; (void)a;
    return NAN;
}

/* ------------------------------------------------------------------ */
/* matmul<T> (k_quants.rs:2284-2331) and qmatmul_generic_f32           */
/* ------------------------------------------------------------------ */

static float vec_dot_any(int t, size_t k, const void *w, const void *a, int use_avx2) {
    switch (t) {
    case FO_Q4K:
        return use_avx2 ? fo_vec_dot_q4k_avx2(k, (const fo_block_q4k *)w, (const fo_block_q8k *)a)
                        : fo_vec_dot_q4k_unopt(k, (const fo_block_q4k *)w, (const fo_block_q8k *)a);
    case FO_Q6K:
        return use_avx2 ? fo_vec_dot_q6k_avx2(k, (const fo_block_q6k *)w, (const fo_block_q8k *)a)
                        : fo_vec_dot_q6k_unopt(k, (const fo_block_q6k *)w, (const fo_block_q8k *)a);
    case FO_Q8_0:
        return use_avx2 ? fo_vec_dot_q8_0_avx2(k, (const fo_block_q8_0 *)w, (const fo_block_q8_0 *)a)
                        : fo_vec_dot_q8_0_unopt(k, (const fo_block_q8_0 *)w, (const fo_block_q8_0 *)a);
    default: return NAN;
    }
}

int fo_matmul(int t, size_t m, size_t k, size_t n, const float *x, const void *w, float *y,
              int use_avx2, int threads) {
    size_t bs = fo_block_size(t);
    if (bs == 0 || t == FO_Q8K) return 3;
    if (k % bs) return 2;
    if (use_avx2 && !fo_have_avx2()) return 3;
    int vt = (t == FO_Q8_0) ? FO_Q8_0 : FO_Q8K;
    size_t kb = k / bs;
    size_t wts = fo_type_size(t), ats = fo_type_size(vt);
    unsigned char *lhs = (unsigned char *)calloc(m * kb + 1, ats);
    if (!lhs) return 5;
    for (size_t r = 0; r < m; r++) { /* activation rows are quantized sequentially */
        if (vt == FO_Q8K) fo_quantize_q8k(x + r * k, k, (fo_block_q8k *)(lhs + r * kb * ats));
        else fo_quantize_q8_0(x + r * k, k, (fo_block_q8_0 *)(lhs + r * kb * ats));
    }
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
#endif
    for (size_t r = 0; r < m; r++) {
        const unsigned char *arow = lhs + r * kb * ats;
        float *yrow = y + r * n;
        /* rayon with_min_len(128)/with_max_len(512): columns in chunks; the
         * per-column arithmetic does not depend on the split. */
#pragma omp parallel for schedule(dynamic, 256) num_threads(nt)
        for (size_t c = 0; c < n; c++)
            yrow[c] = vec_dot_any(t, k, (const unsigned char *)w + c * kb * wts, arow, use_avx2);
    }
    free(lhs);
    return 0;
}

int fo_qmatmul_bytes(int t, size_t batch, size_t m, size_t n, size_t k, const float *act,
                     size_t act_bytes, const void *w, size_t w_bytes, float *out, size_t out_bytes,
                     int use_avx2, int threads) {
    size_t bs = fo_block_size(t);
    if (bs == 0 || t == FO_Q8K) return 3;
    if (k % bs) return 2;
    if (w_bytes != n * (k / bs) * fo_type_size(t)) return 2;
    if (act_bytes != batch * m * k * 4) return 2;
    if (out_bytes != batch * m * n * 4) return 2;
    if (batch == 0 || m == 0 || n == 0) return 0;
    for (size_t b = 0; b < batch; b++) {
        int rc = fo_matmul(t, m, k, n, act + b * m * k, w, out + b * m * n, use_avx2, threads);
        if (rc) return rc;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* MoE                                                                  */
/* ------------------------------------------------------------------ */

void fo_moe_route(const float *logits, size_t t, size_t e, size_t topk, int32_t *ids, float *w,
                  int32_t *expert_offsets, int32_t *sorted_token_ids, int32_t *sorted_slot) {
    float *work = (float *)malloc(e * sizeof(float));
    for (size_t r = 0; r < t; r++) {
        memcpy(work, logits + r * e, e * sizeof(float));
        float picked[64];
        /* lazy_nn/moe.rs:106-118: k rounds of argmax (first index wins,
         * byte_kernels.rs:8246-8261) then mask the pick with -1e30. */
        for (size_t s = 0; s < topk; s++) {
            size_t best = 0;
            float bv = work[0]; /* the first slot is taken unconditionally */
            for (size_t j = 1; j < e; j++)
                if (work[j] > bv) {
                    bv = work[j];
                    best = j;
                }
            ids[r * topk + s] = (int32_t)best;
            picked[s] = logits[r * e + best];
            work[best] += -1e30f;
        }
        /* softmax_last_dim_f32 (byte_kernels.rs:2259-2305) over the picks */
        float mx = picked[0];
        for (size_t s = 1; s < topk; s++)
            if (picked[s] > mx) mx = picked[s];
        float sum = 0.0f, ex[64];
        for (size_t s = 0; s < topk; s++) {
            ex[s] = expf(picked[s] - mx);
            sum += ex[s];
        }
        float inv = 1.0f / sum;
        for (size_t s = 0; s < topk; s++) w[r * topk + s] = ex[s] * inv;
    }
    free(work);
    /* build_expert_batches (moe_routing.rs:334-360): experts ascending,
     * tokens ascending within each expert. */
    for (size_t j = 0; j <= e; j++) expert_offsets[j] = 0;
    for (size_t i = 0; i < t * topk; i++) expert_offsets[ids[i] + 1]++;
    for (size_t j = 0; j < e; j++) expert_offsets[j + 1] += expert_offsets[j];
    int32_t *fill = (int32_t *)calloc(e, sizeof(int32_t));
    for (size_t r = 0; r < t; r++)
        for (size_t s = 0; s < topk; s++) {
            int32_t ex_id = ids[r * topk + s];
            int32_t pos = expert_offsets[ex_id] + fill[ex_id]++;
            sorted_token_ids[pos] = (int32_t)r;
            if (sorted_slot) sorted_slot[pos] = (int32_t)(r * topk + s);
        }
    free(fill);
}

int fo_moe_ffn(int t, size_t ntok, size_t d, size_t ffn, size_t ne, size_t topk, const float *x,
               const int32_t *ids, const float *w, const void *w_gate, const void *w_up,
               const void *w_down, float *out, int use_avx2, int threads) {
    size_t bs = fo_block_size(t), ts = fo_type_size(t);
    if (bs == 0 || d % bs || ffn % bs) return 2;
    size_t gate_bytes = ffn * (d / bs) * ts, down_bytes = d * (ffn / bs) * ts;
    memset(out, 0, ntok * d * sizeof(float));
    float *xs = (float *)malloc(ntok * d * sizeof(float));
    float *g = (float *)malloc(ntok * ffn * sizeof(float));
    float *u = (float *)malloc(ntok * ffn * sizeof(float));
    float *yd = (float *)malloc(ntok * d * sizeof(float));
    int32_t *sel = (int32_t *)malloc(ntok * sizeof(int32_t));
    float *gw = (float *)malloc(ntok * sizeof(float));
    int rc = 0;
    for (size_t ex = 0; ex < ne && !rc; ex++) {
        size_t cnt = 0;
        for (size_t r = 0; r < ntok; r++)
            for (size_t s = 0; s < topk; s++)
                if ((size_t)ids[r * topk + s] == ex) {
                    sel[cnt] = (int32_t)r;
                    gw[cnt] = w[r * topk + s];
                    cnt++;
                }
        if (!cnt) continue;
        for (size_t i = 0; i < cnt; i++) memcpy(xs + i * d, x + (size_t)sel[i] * d, d * sizeof(float));
        rc |= fo_matmul(t, cnt, d, ffn, xs, (const char *)w_gate + ex * gate_bytes, g, use_avx2, threads);
        rc |= fo_matmul(t, cnt, d, ffn, xs, (const char *)w_up + ex * gate_bytes, u, use_avx2, threads);
        for (size_t i = 0; i < cnt * ffn; i++) {
            float gv = g[i];
            g[i] = gv / (1.0f + expf(-gv)) * u[i];
        }
        rc |= fo_matmul(t, cnt, ffn, d, g, (const char *)w_down + ex * down_bytes, yd, use_avx2, threads);
        for (size_t i = 0; i < cnt; i++)
            for (size_t c = 0; c < d; c++) out[(size_t)sel[i] * d + c] += yd[i * d + c] * gw[i];
    }
    free(xs); free(g); free(u); free(yd); free(sel); free(gw);
    return rc;
}

/* ------------------------------------------------------------------ */
/* LLaMA decoder pieces                                                 */
/* ------------------------------------------------------------------ */

void fo_rms_norm(const float *x, const float *gain, size_t rows, size_t dim, float eps, float *y) {
    const float inv_n = 1.0f / (float)dim;
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * dim;
        float sum_sq = 0.0f;
        for (size_t j = 0; j < dim; j++) sum_sq += xr[j] * xr[j];
        const float mean_sq = sum_sq * inv_n;
        const float rms_inv = 1.0f / sqrtf(mean_sq + eps);
        for (size_t j = 0; j < dim; j++) {
            const float nrm = xr[j] * rms_inv; /* normalized tensor, then the gain multiply */
            y[r * dim + j] = nrm * gain[j];
        }
    }
}

void fo_rope_tables(double base, size_t start_pos, size_t seq, size_t head_dim, float *cos_t, float *sin_t) {
    const size_t half = head_dim / 2;
    for (size_t p = 0; p < seq; p++) {
        const double pos = (double)(start_pos + p);
        for (size_t i = 0; i < half; i++) {
            const double freq = pow(base, -2.0 * (double)i / (double)head_dim);
            const double theta = pos * freq;
            const float c = (float)cos(theta), s = (float)sin(theta);
            cos_t[p * head_dim + i] = c;
            cos_t[p * head_dim + i + half] = c;
            sin_t[p * head_dim + i] = s;
            sin_t[p * head_dim + i + half] = s;
        }
    }
}

void fo_rope(const float *x, const float *cos_t, const float *sin_t, size_t outer, size_t seq, size_t head_dim,
             float *y) {
    const size_t h = head_dim / 2;
    for (size_t o = 0; o < outer; o++)
        for (size_t s = 0; s < seq; s++) {
            const float *xr = x + (o * seq + s) * head_dim;
            float *yr = y + (o * seq + s) * head_dim;
            const float *c = cos_t + s * head_dim, *sn = sin_t + s * head_dim;
            for (size_t i = 0; i < h; i++) {
                const float lo = xr[i], hi = xr[i + h];
                yr[i] = lo * c[i] - hi * sn[i];
                yr[i + h] = hi * c[i + h] + lo * sn[i + h];
            }
        }
}

void fo_attention_decode(const float *q, const float *k, const float *v, size_t heads, size_t n_ctx, size_t stride,
                         size_t head_dim, float scale, float *out) {
    float *sc = (float *)malloc((n_ctx ? n_ctx : 1) * sizeof(float));
    for (size_t h = 0; h < heads; h++) {
        const float *qh = q + h * head_dim;
        const float *kh = k + h * stride * head_dim, *vh = v + h * stride * head_dim;
        for (size_t j = 0; j < n_ctx; j++) {
            float d = 0.0f;
            for (size_t e = 0; e < head_dim; e++) d += qh[e] * kh[j * head_dim + e];
            sc[j] = d * scale;
        }
        float mx = sc[0];
        for (size_t j = 1; j < n_ctx; j++)
            if (sc[j] > mx) mx = sc[j];
        float sum = 0.0f;
        for (size_t j = 0; j < n_ctx; j++) {
            sc[j] = expf(sc[j] - mx);
            sum += sc[j];
        }
        const float inv = 1.0f / sum;
        for (size_t j = 0; j < n_ctx; j++) sc[j] *= inv;
        for (size_t e = 0; e < head_dim; e++) {
            float o = 0.0f;
            for (size_t j = 0; j < n_ctx; j++) o += sc[j] * vh[j * head_dim + e];
            out[h * head_dim + e] = o;
        }
    }
    free(sc);
}

size_t fo_argmax(const float *x, size_t n) {
    size_t best = 0;
    float bv = n ? x[0] : 0.0f;
    for (size_t i = 1; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    return best;
}
