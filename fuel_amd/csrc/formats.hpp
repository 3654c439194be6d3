// Per-lane block-dot building blocks shared by the mat-vec kernels and the
// integer tap.  A weight block is handled by LPB consecutive lanes; lane c of
// the block:
//   load(blk, c)          issues the global loads of its share of the block
//                          (raw registers, no use of the data yet), and
//   dot(raw, act, c, ...) turns them into the integer partial sums
//                          (isum, msum) and the block's f32 d / dmin.
// Splitting the two lets a kernel keep the next row's loads in flight while it
// computes the current one.  The integer partials of the LPB lanes of a block
// add up exactly to the integer sums of vec_dot_unopt (k_quants.rs:1388-1468,
// 1946-2003, 674-692).
#pragma once

#include "common.hpp"

namespace frq {

// ------------------------------------------------------------------------
// Q4K (144 B, 16-byte multiple): 4 lanes per superblock.  Lane c owns quant
// bytes qs[32c..32c+32): low nibbles = elements 64c..64c+31 (sub-block 2c),
// high nibbles = 64c+32..64c+63 (sub-block 2c+1)  (k_quants.rs:1603-1620).
// ------------------------------------------------------------------------
struct Q4K {
    static constexpr int LPB = 4;
    static constexpr int BYTES = Q4K_BYTES;
    static constexpr int ELEMS = QK_K;
    static constexpr int ACT = GGML_Q8K;
    // LDS bytes per activation superblock: lane c of block b reads 64
    // contiguous bytes at 64c, so with 16 lanes served per cycle (blocks
    // b..b+3) the 68-dword stride puts the 16 reads of a cycle on disjoint
    // bank quads (4b + 16c mod 64)
    static constexpr int QSTRIDE = QK_K + 16;
    struct Act {
        uint4 a[4];  // q8 of elements 64c + 0..63
        int bs_lo;   // bsums[4c] + bsums[4c+1]
        int bs_hi;   // bsums[4c+2] + bsums[4c+3]
        float d;
    };
    struct Raw {
        uint4 hd, q0, q1;
    };
    // Activation slice of block b: quants `qstride` bytes apart per superblock,
    // d [KB], bsums [KB][16].
    __device__ static void load_act(const int8_t* qs, int qstride, const float* dv, const int16_t* bsums, int b,
                                    int c, Act& r) {
        const uint4* q = reinterpret_cast<const uint4*>(qs + (size_t)b * qstride + 64 * c);
        r.a[0] = q[0];
        r.a[1] = q[1];
        r.a[2] = q[2];
        r.a[3] = q[3];
        const int16_t* bs = bsums + (size_t)b * 16 + 4 * c;
        r.bs_lo = (int)bs[0] + (int)bs[1];
        r.bs_hi = (int)bs[2] + (int)bs[3];
        r.d = dv[b];
    }
    __device__ static void load(const uint8_t* blk, int c, Raw& r) {
        r.hd = *reinterpret_cast<const uint4*>(blk);
        r.q0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * c);
        r.q1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * c);
    }
    // The same pieces through a buffer resource of the row (a scalar base and
    // size) at a 32-bit offset: qmv_load_row's long rows.
    static constexpr bool BUF = true;
    __device__ static void load_buf(__amdgpu_buffer_rsrc_t R, uint32_t off, int c, Raw& r) {
        r.hd = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(R, off, 0, 0));
        r.q0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(R, off + 16u + 32u * (uint32_t)c, 0, 0));
        r.q1 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(R, off + 32u + 32u * (uint32_t)c, 0, 0));
    }
    __device__ static void dot(const Raw& r, const Act& x, int c, int& isum, int& msum, float& dw, float& dmw) {
        // 12 packed bytes -> 8 six-bit scales and 8 mins (get_scale_min_k4,
        // utils.rs:50-60) as four words of bytes.
        const uint32_t s0 = r.hd.y, s1 = r.hd.z, s2 = r.hd.w;
        const uint32_t sc_a = s0 & 0x3f3f3f3fu;                                              // scales 0..3
        const uint32_t sc_b = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);         // scales 4..7
        const uint32_t mn_a = s1 & 0x3f3f3f3fu;                                              // mins 0..3
        const uint32_t mn_b = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);  // mins 4..7
        const uint32_t scw = c < 2 ? sc_a : sc_b;
        const uint32_t mnw = c < 2 ? mn_a : mn_b;
        const uint32_t sh = 16u * (uint32_t)(c & 1);
        const int sc_lo = (int)((scw >> sh) & 0xffu), sc_hi = (int)((scw >> (sh + 8)) & 0xffu);
        const int m_lo = (int)((mnw >> sh) & 0xffu), m_hi = (int)((mnw >> (sh + 8)) & 0xffu);
        const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t alo[8] = {x.a[0].x, x.a[0].y, x.a[0].z, x.a[0].w, x.a[1].x, x.a[1].y, x.a[1].z, x.a[1].w};
        const uint32_t ahi[8] = {x.a[2].x, x.a[2].y, x.a[2].z, x.a[2].w, x.a[3].x, x.a[3].y, x.a[3].z, x.a[3].w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo = dot4(w[i] & 0x0f0f0f0fu, alo[i], lo);
            hi = dot4((w[i] >> 4) & 0x0f0f0f0fu, ahi[i], hi);
        }
        // |lo|, |hi| < 2^16 and the 6-bit scales fit 24-bit multiplies exactly
        isum = __mul24(sc_lo, lo) + __mul24(sc_hi, hi);
        msum = __mul24(m_lo, x.bs_lo) + __mul24(m_hi, x.bs_hi);
        dw = f16_to_f32(r.hd.x & 0xffffu);
        dmw = f16_to_f32(r.hd.x >> 16);
    }
};

// ------------------------------------------------------------------------
// Q6K (210 B, only 2-byte aligned): 4 lanes per superblock.  Lane c -> half
// hh = c>>1 (elements 128hh..+127) and column offset l0 = 16*(c&1); it owns
// elements 128hh + 32qd + l0 + [0,16) for qd = 0..3 from ql[64hh+l0..+16]
// (qd 0 low / qd 2 high nibbles), ql[64hh+32+l0..+16] (qd 1 / 3) and
// qh[32hh+l0..+16] (2 bits per qd)  (k_quants.rs:2170-2186); the scale of qd
// is scales[8hh + 2qd + (c&1)].  Each 16-byte piece is one unaligned load.
// ------------------------------------------------------------------------
struct Q6K {
    static constexpr bool BUF = false;  // (row loads through plain pointers only)
    static constexpr int LPB = 4;
    static constexpr int BYTES = Q6K_BYTES;
    static constexpr int ELEMS = QK_K;
    static constexpr int ACT = GGML_Q8K;
    // lane c reads 16 bytes at 128 (c >> 1) + 16 (c & 1) + 32 qd: dword quads
    // {0, 4, 32, 36} + stride * b.  A 68-dword stride (Q4K's) overlaps them for
    // neighbouring blocks (two-way bank conflicts); 72 dwords (8 mod 64) keeps
    // the 16 quads of a cycle disjoint
    static constexpr int QSTRIDE = QK_K + 32;
    struct Act {
        uint4 a[4];  // q8 of the lane's 4 groups of 16
        int bs[4];   // bsums of those groups
        float d;
    };
    struct Raw {
        uint4 la, lb, qh;
        uint2 sc;  // scales[8hh..8hh+8)
        uint32_t dbits;
    };
    __device__ static void load_act(const int8_t* qs, int qstride, const float* dv, const int16_t* bsums, int b,
                                    int c, Act& r) {
        const int hh = c >> 1, l0 = 16 * (c & 1);
        const int8_t* q = qs + (size_t)b * qstride + 128 * hh + l0;
        // bsums 8hh .. 8hh+7 in one 16-byte read (four 2-byte reads, 32 bytes
        // apart per block, put four blocks on one bank); group 8hh + (c&1) + 2qd
        // is the low (c even) or high half of word qd
        const uint4 bq = *reinterpret_cast<const uint4*>(bsums + (size_t)b * 16 + 8 * hh);
        const uint32_t bw[4] = {bq.x, bq.y, bq.z, bq.w};
        const uint32_t bsh = 16u * (uint32_t)(c & 1);
#pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            r.a[qd] = *reinterpret_cast<const uint4*>(q + 32 * qd);
            r.bs[qd] = (int)(int16_t)(uint16_t)(bw[qd] >> bsh);
        }
        r.d = dv[b];
    }
    __device__ static void load(const uint8_t* blk, int c, Raw& r) {
        const int hh = c >> 1, l0 = 16 * (c & 1);
        r.la = load16_u(blk + 64 * hh + l0);
        r.lb = load16_u(blk + 64 * hh + 32 + l0);
        r.qh = load16_u(blk + 128 + 32 * hh + l0);
        r.sc = load8_u(blk + 192 + 8 * hh);
        r.dbits = load_u16(blk + 208);
    }
    __device__ static void dot(const Raw& r, const Act& x, int c, int& isum, int& msum, float& dw, float& dmw) {
        const uint32_t wa[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
        const uint32_t wb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
        const uint32_t wh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        const uint32_t scx = r.sc.x, scy = r.sc.y;
        const uint32_t a0[4] = {x.a[0].x, x.a[0].y, x.a[0].z, x.a[0].w};
        const uint32_t a1[4] = {x.a[1].x, x.a[1].y, x.a[1].z, x.a[1].w};
        const uint32_t a2[4] = {x.a[2].x, x.a[2].y, x.a[2].z, x.a[2].w};
        const uint32_t a3[4] = {x.a[3].x, x.a[3].y, x.a[3].z, x.a[3].w};
        // Unsigned 6-bit codes u in [0, 64): sum (u-32)*q8 = dot(u, q8) - 32*bsum.
        int p0 = 0, p1 = 0, p2 = 0, p3 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t u0 = (wa[i] & 0x0f0f0f0fu) | ((wh[i] & 0x03030303u) << 4);
            const uint32_t u1 = (wb[i] & 0x0f0f0f0fu) | (((wh[i] >> 2) & 0x03030303u) << 4);
            const uint32_t u2 = ((wa[i] >> 4) & 0x0f0f0f0fu) | (((wh[i] >> 4) & 0x03030303u) << 4);
            const uint32_t u3 = ((wb[i] >> 4) & 0x0f0f0f0fu) | (((wh[i] >> 6) & 0x03030303u) << 4);
            p0 = dot4(u0, a0[i], p0);
            p1 = dot4(u1, a1[i], p1);
            p2 = dot4(u2, a2[i], p2);
            p3 = dot4(u3, a3[i], p3);
        }
        p0 -= 32 * x.bs[0];
        p1 -= 32 * x.bs[1];
        p2 -= 32 * x.bs[2];
        p3 -= 32 * x.bs[3];
        // scales byte j = 2qd + (c&1) of the 8-byte window, sign-extended
        const uint32_t sel = (uint32_t)(c & 1) * 8u;
        const int sc0 = (int)(int8_t)((scx >> sel) & 0xffu);
        const int sc1 = (int)(int8_t)((scx >> (sel + 16)) & 0xffu);
        const int sc2 = (int)(int8_t)((scy >> sel) & 0xffu);
        const int sc3 = (int)(int8_t)((scy >> (sel + 16)) & 0xffu);
        // |p| <= 32*128*16 < 2^23: exact in 24-bit multiplies
        isum = __mul24(sc0, p0) + __mul24(sc1, p1) + __mul24(sc2, p2) + __mul24(sc3, p3);
        msum = 0;
        dw = f16_to_f32(r.dbits);
        dmw = 0.0f;
    }
};

// ------------------------------------------------------------------------
// Q8_0 (34 B, 2-byte aligned): 2 lanes per block; lane c owns qs[16c..16c+16).
// Its 16 bytes start 2 bytes past a 4-byte boundary in every other block; a
// 16-byte load from there runs a third slower than a dword-aligned one
// (4096x32000: 41.5 against 29.1 us), so the lane loads the dword-aligned
// 16 bytes at or below its piece plus, when they fall 2 bytes short, the 2
// bytes after them, and funnel-shifts the words into place (v_alignbyte) when
// it reduces the block.  (Weights are 4-byte aligned: every piece starts at
// 0 or 2 mod 4.)
// ------------------------------------------------------------------------
struct Q80 {
    static constexpr bool BUF = false;  // (row loads through plain pointers only)
    static constexpr int LPB = 2;
    static constexpr int BYTES = Q8_0_BYTES;
    static constexpr int ELEMS = QK8_0;
    static constexpr int ACT = GGML_Q8_0;
    static constexpr int QSTRIDE = 0;  // (Q8_0 rows: the blocks packed, 32 bytes apart)
    struct Act {
        uint4 a;
        float d;
    };
    struct Raw {
        uint4 q;         // the dword-aligned 16 bytes at or below the piece
        uint32_t tail;   // the 2 bytes after them (a shifted piece only)
        uint32_t sh;     // the piece's byte offset in q: 0 or 2
        uint32_t dbits;
    };
    __device__ static void load_act(const int8_t* qs, int qstride, const float* dv, const int16_t*, int b, int c,
                                    Act& r) {
        r.a = *reinterpret_cast<const uint4*>(qs + (size_t)b * qstride + 16 * c);
        r.d = dv[b];
    }
    __device__ static void load(const uint8_t* blk, int c, Raw& r) {
        const uint8_t* p = blk + 2 + 16 * c;
        r.sh = (uint32_t)((uintptr_t)p & 3);
        const uint8_t* a = p - r.sh;
        r.q = *reinterpret_cast<const uint4*>(a);
        // (bytes a+16, a+17 = p+14, p+15 when shifted; otherwise the block's
        // d again: every address stays inside the block)
        r.tail = load_u16(r.sh ? a + 16 : blk);
        r.dbits = load_u16(blk);
    }
    __device__ static void dot(const Raw& r, const Act& x, int, int& isum, int& msum, float& dw, float& dmw) {
        const uint32_t q[4] = {__builtin_amdgcn_alignbyte(r.q.y, r.q.x, r.sh),
                               __builtin_amdgcn_alignbyte(r.q.z, r.q.y, r.sh),
                               __builtin_amdgcn_alignbyte(r.q.w, r.q.z, r.sh),
                               __builtin_amdgcn_alignbyte(r.tail, r.q.w, r.sh)};
        int s = 0;
        s = dot4(q[0], x.a.x, s);
        s = dot4(q[1], x.a.y, s);
        s = dot4(q[2], x.a.z, s);
        s = dot4(q[3], x.a.w, s);
        isum = s;
        msum = 0;
        dw = f16_to_f32(r.dbits);
        dmw = 0.0f;
    }
};

}  // namespace frq
