// Format policies of the int8-MFMA kernels that read the weight blocks
// straight into registers (mmq_skinny.hip):
// per 256-element unit, the lane's raw loads (the one-row mat-vec's lane c
// loads for that column's block, formats.hpp), the activation byte offset of
// its K slots at MFMA step t, and the MFMAs + f32 step into facc[RT][4].  The
// K slots of a step are ordered to match those loads (a dot product does not
// depend on the order of K as long as A and B agree): lane group c of step t
// holds elements
//   Q4_K  64c + 16t + [0,16)                    (nibbles of its two 16-byte qs pieces)
//   Q6_K  128(c>>1) + 32t + 16(c&1) + [0,16)    (its ql / qh pieces, code t)
//   Q8_0  32j + 8c + [0,8) of block j           (v_mfma_i32_16x16x32_i8, one block per MFMA)
// and `a(rt, t)` supplies the A fragment (16 bytes of those elements of the
// lane's activation row in row tile rt).  Integer sums per superblock / block
// are exact:
//   Q4_K  isum = 8*(X.Ba) + X.Bb, msum = X.Bm  (sc = 8a + b; mins broadcast),
//   Q6_K  isum = 128*(X.Wh) + X.Wl            (w = (q-32)*sc = 128 wh + wl),
//   Q8_0  isum = X.Q,
// then one f32 step per superblock (block): y += d_x * (d*isum - dmin*msum).
#pragma once

#include "common.hpp"
#include "formats.hpp"
#include "mfma.hpp"

namespace frq {

constexpr int SK_UNIT = QK_K;  // elements per unit of the K loop

typedef long i64;

// ---- format policies: per unit, the lane's raw loads, its A fragment
// offsets and the MFMAs + f32 step into facc[RT][4] ----

struct SkQ4K {
    using Raw = Q4K::Raw;
    static constexpr int BYTES = Q4K_BYTES;
    static constexpr int ACT = GGML_Q8K;
    static constexpr int NA = 4;  // A fragments per row tile and unit (16 bytes each)
    __device__ static void load(const uint8_t* row, int u, int c, Raw& r) { Q4K::load(row + (size_t)u * BYTES, c, r); }
    __device__ static uint32_t aoff(int c, int t) { return 64u * c + 16u * t; }
    template <int RT, class GetA>
    __device__ static void unit(const Raw& r, GetA a, int c, const float (&dx)[RT][4], float (&facc)[RT][4]) {
        const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w;
        const uint32_t sc_a = s0 & 0x3f3f3f3fu;
        const uint32_t sc_b = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_a = s1 & 0x3f3f3f3fu;
        const uint32_t mn_b = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
        const uint32_t scw = c < 2 ? sc_a : sc_b, mnw = c < 2 ? mn_a : mn_b;
        const uint32_t sh = 16u * (uint32_t)(c & 1);
        const uint32_t sc2[2] = {(scw >> sh) & 0xffu, (scw >> (sh + 8)) & 0xffu};  // sub-blocks 2c, 2c+1
        const uint32_t mn2[2] = {(mnw >> sh) & 0xffu, (mnw >> (sh + 8)) & 0xffu};
        const uint32_t q[2][4] = {{r.q0.x, r.q0.y, r.q0.z, r.q0.w}, {r.q1.x, r.q1.y, r.q1.z, r.q1.w}};
        v4i acc[RT][3];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int hi = t >> 1;  // t = 0, 1: low nibbles (sub-block 2c); 2, 3: high (2c+1)
            const uint32_t* w = q[t & 1];
            const uint32_t fa = sc2[hi] >> 3, fb = sc2[hi] & 7u;
            uint32_t nb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) nb[i] = (w[i] >> (4 * hi)) & 0x0f0f0f0fu;
            const v4i ba = v4i{bytes_times(nb[0], fa), bytes_times(nb[1], fa), bytes_times(nb[2], fa),
                               bytes_times(nb[3], fa)};
            const v4i bb = v4i{bytes_times(nb[0], fb), bytes_times(nb[1], fb), bytes_times(nb[2], fb),
                               bytes_times(nb[3], fb)};
            const int mb = (int)(mn2[hi] * 0x01010101u);
            const v4i bm = v4i{mb, mb, mb, mb};
            const v4i zero = v4i{0, 0, 0, 0};
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const v4i av = a(rt, t);
                acc[rt][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, ba, t == 0 ? zero : acc[rt][0], 0, 0, 0);
                acc[rt][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bb, t == 0 ? zero : acc[rt][1], 0, 0, 0);
                acc[rt][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bm, t == 0 ? zero : acc[rt][2], 0, 0, 0);
            }
        }
        const float d = f16_to_f32(r.hd.x & 0xffffu), dmin = f16_to_f32(r.hd.x >> 16);
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int isum = 8 * acc[rt][0][i] + acc[rt][1][i];
                facc[rt][i] = fmaf(dx[rt][i], fmaf(-dmin, (float)acc[rt][2][i], d * (float)isum), facc[rt][i]);
            }
    }
};

struct SkQ6K {
    using Raw = Q6K::Raw;
    static constexpr int BYTES = Q6K_BYTES;
    static constexpr int ACT = GGML_Q8K;
    static constexpr int NA = 4;
    __device__ static void load(const uint8_t* row, int u, int c, Raw& r) { Q6K::load(row + (size_t)u * BYTES, c, r); }
    __device__ static uint32_t aoff(int c, int t) { return 128u * (c >> 1) + 32u * t + 16u * (c & 1); }
    template <int RT, class GetA>
    __device__ static void unit(const Raw& r, GetA a, int c, const float (&dx)[RT][4], float (&facc)[RT][4]) {
        const uint32_t la[4] = {r.la.x, r.la.y, r.la.z, r.la.w}, lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
        const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        const uint32_t sel = 8u * (uint32_t)(c & 1);
        v4i acc[RT][2];
#pragma unroll
        for (int t = 0; t < 4; t++) {  // code t: ql nibble t>>1 of la (t even) / lb (t odd), qh bits 2t
            const uint32_t scw = t < 2 ? r.sc.x : r.sc.y;
            const int sc = (int)(int8_t)((scw >> (16u * (uint32_t)(t & 1) + sel)) & 0xffu);  // scales[8hh + 2t + (c&1)]
            const uint32_t f = (uint32_t)sc & 0xffffu, cst = (uint32_t)(-32 * sc) & 0xffffu;
            const uint32_t sc16 = f | (f << 16), c16 = cst | (cst << 16);
            const uint32_t* l = (t & 1) ? lb : la;
            int wl[4], wh[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t u = ((l[i] >> (4 * (t >> 1))) & 0x0f0f0f0fu) | (((qh[i] >> (2 * t)) & 0x03030303u) << 4);
                q6_planes(u, sc16, c16, wl[i], wh[i]);
            }
            const v4i bh = v4i{wh[0], wh[1], wh[2], wh[3]}, bl = v4i{wl[0], wl[1], wl[2], wl[3]};
            const v4i zero = v4i{0, 0, 0, 0};
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const v4i av = a(rt, t);
                acc[rt][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bh, t == 0 ? zero : acc[rt][0], 0, 0, 0);
                acc[rt][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bl, t == 0 ? zero : acc[rt][1], 0, 0, 0);
            }
        }
        const float d = f16_to_f32(r.dbits);
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int isum = 128 * acc[rt][0][i] + acc[rt][1][i];
                facc[rt][i] = fmaf(dx[rt][i], d * (float)isum, facc[rt][i]);
            }
    }
};

// Q8_0: a unit is eight 34-byte blocks; lane group c holds bytes 8c..8c+7 of
// each block's quants and the block's f16 d.  The unit starts on a 16-byte
// boundary (rows of K/32 blocks with K a multiple of 256, weights 4-byte
// aligned), so the pieces of the even blocks start 2 bytes past a dword
// boundary: those load the dword-aligned 8 bytes below plus the 2 bytes after
// them and funnel-shift (an 8-byte load 2 bytes off a dword boundary runs far
// slower than an aligned one).
struct SkQ80 {
    struct Raw {
        uint2 q[8];
        uint32_t tail[4];  // even blocks: bytes 6, 7 of the piece
        uint32_t dbits[8];
    };
    static constexpr int BYTES = 8 * Q8_0_BYTES;
    static constexpr int ACT = GGML_Q8_0;
    static constexpr int NA = 4;  // 16-byte A loads: blocks (2i, 2i+1)'s 8-byte slices
    __device__ static void load(const uint8_t* row, int u, int c, Raw& r) {
        const uint8_t* b = row + (size_t)u * BYTES;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint8_t* p = b + j * Q8_0_BYTES + 2 + 8 * c;
            if (j & 1) {
                r.q[j] = *reinterpret_cast<const uint2*>(p);
            } else {
                r.q[j] = *reinterpret_cast<const uint2*>(p - 2);
                r.tail[j >> 1] = load_u16(p + 6);
            }
            r.dbits[j] = load_u16(b + j * Q8_0_BYTES);
        }
    }
    // A fragment i (16 bytes) = blocks 2i and 2i+1's slices 8c..8c+7: two
    // 8-byte pieces 32 bytes apart; loaded as two halves by the kernel
    __device__ static uint32_t aoff(int c, int t) { return 64u * t + 8u * c; }
    // dx: the activation scales of the lane's output rows, d [M][K/32] (the
    // unit's blocks are read per block: 4 per row tile)
    template <int RT, class GetA>
    __device__ static void unit(const Raw& r, GetA a, int c, const float* const (&dx)[RT][4],
                                float (&facc)[RT][4]) {
        (void)c;
        const v4i zero = v4i{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t lo = r.q[j].x, hi = r.q[j].y;
            if (!(j & 1)) {
                lo = __builtin_amdgcn_alignbyte(r.q[j].y, r.q[j].x, 2);
                hi = __builtin_amdgcn_alignbyte(r.tail[j >> 1], r.q[j].y, 2);
            }
            const i64 bq = (i64)(((unsigned long long)hi << 32) | lo);
            const float dw = f16_to_f32(r.dbits[j]);
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const v4i av = a(rt, j >> 1);
                const i64 aq = (j & 1) ? (i64)(((unsigned long long)(uint32_t)av[3] << 32) | (uint32_t)av[2])
                                       : (i64)(((unsigned long long)(uint32_t)av[1] << 32) | (uint32_t)av[0]);
                const v4i s = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, bq, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) facc[rt][i] = fmaf(dw * dx[rt][i][j], (float)s[i], facc[rt][i]);
            }
        }
    }
};

}  // namespace frq
