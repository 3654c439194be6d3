// Per-row building blocks of the quantized mat-vec kernels (mmvq.hip,
// mmvq_multi.hip): launch sizes, the unconditional loads of one weight row
// into registers and the row's dot product against an LDS activation row.
#pragma once

#include "common.hpp"
#include "formats.hpp"


namespace frq {

// Workgroup size for many rows: 1024 threads while a row's raw weight
// registers stay small (<= 36 dwords: the kernel then fits the 128 VGPRs a
// 1024-thread workgroup allows), 512 up to 40 dwords, else 256.  Fewer,
// larger workgroups quantize the activation row fewer times per CU (measured:
// 4096x11008 Q4_K 7.8 -> 7.5 us, Q6_K 12.4 -> 11.0 us; 256 threads is slower).
template <class F, int SPL>
constexpr int qmv_wg() {
    constexpr int raw = SPL * (int)(sizeof(typename F::Raw) / 4);
    return raw <= 36 ? 1024 : raw <= 40 ? 512 : 256;
}

// Workgroup size for few rows (about two per wavefront at one workgroup per
// CU): as large as the register budget allows, so that one workgroup per CU
// quantizes the activation row once for all its wavefronts (1024 threads
// need <= 128 VGPRs, 512 threads <= 256).
template <class F, int SPL>
constexpr int qmv_wg_big() {
    constexpr int raw = SPL * (int)(sizeof(typename F::Raw) / 4);
    return raw <= 36 ? 1024 : raw <= 48 ? 512 : qmv_wg<F, SPL>();
}

// The loads are unconditional (a slot past the row's last block re-reads that
// block; qmv_row skips it): with no branch around them the in-order vmcnt
// counter can wait for one row while the next row's loads stay in flight.
template <class F, int SPL>
__device__ __forceinline__ void qmv_load_row(const uint8_t* __restrict__ wr, int gi, int c, int KB,
                                             typename F::Raw (&r)[SPL]) {
    constexpr int BPW = 64 / F::LPB;
    if constexpr (F::BUF && SPL >= 3) {
        // Rows of three or more slots (K > 8192) through a buffer resource of
        // the row: a scalar base, 32-bit vector offsets that stay the same
        // from row to row, no vector address arithmetic per row (Q4_K
        // 11008x4096 8.55 -> 8.38 us, 4096 rows of K = 12288 9.06 -> 8.90;
        // for one-slot rows it measured slower: 4096x11008 6.74 -> 7.2-7.4,
        // 4096x32000 14.27 -> 14.6-14.7).  The row's size is the record
        // count, so a stray offset reads zeros, not another row; word 3 as
        // gfx9 raw buffers take it.
        const __amdgpu_buffer_rsrc_t R =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wr), (short)0, KB * F::BYTES, 0x00020000);
#pragma unroll
        for (int s = 0; s < SPL; s++) {
            const int b = gi + BPW * s;
            F::load_buf(R, (uint32_t)((b < KB ? b : KB - 1) * F::BYTES), c, r[s]);
        }
    } else {
#pragma unroll
        for (int s = 0; s < SPL; s++) {
            const int b = gi + BPW * s;
            F::load(wr + (size_t)(b < KB ? b : KB - 1) * F::BYTES, c, r[s]);
        }
    }
}

// Marks a row's raw registers as used on every path.  qmv_row skips a slot
// past the row's end with a branch, so after it the compiler counts that
// slot's loads as possibly still in flight, and a ring that reuses the
// registers then waits for everything issued after them (the whole next row)
// before its next loads.  Used after the loads were consumed, this costs no
// instruction and no wait.
template <class F, int SPL>
__device__ __forceinline__ void qmv_settle_row(const typename F::Raw (&r)[SPL]) {
#pragma unroll
    for (int s = 0; s < SPL; s++) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(&r[s]);
#pragma unroll
        for (int i = 0; i < (int)(sizeof(typename F::Raw) / 4); i++) asm volatile("" ::"v"(p[i]));
    }
}

// The lane's activation slices of its block slots, read from LDS once: with
// one activation row they are the same for every weight row, so the rings
// keep them in registers (qmv_row_x) instead of reading them again per row.
// A slot past the row's end reads the last block (never used).
template <class F, int SPL>
__device__ __forceinline__ void qmv_load_acts(const int8_t* s_qs, int qstride, const float* s_d, const int16_t* s_bs,
                                              int gi, int c, int KB, typename F::Act (&xa)[SPL]) {
    constexpr int BPW = 64 / F::LPB;
#pragma unroll
    for (int s = 0; s < SPL; s++) {
        const int b = gi + BPW * s;
        F::load_act(s_qs, qstride, s_d, s_bs, b < KB ? b : KB - 1, c, xa[s]);
    }
}

// qmv_row with the activation slices in registers (the same arithmetic in
// the same order: the same bits).
template <class F, int SPL, int RPW = 1>
__device__ __forceinline__ float qmv_row_x(const typename F::Raw (&r)[SPL], const typename F::Act (&xa)[SPL], int gi,
                                           int c, int KB) {
    constexpr int BPW = 64 / F::LPB;
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < SPL; s++) {
        const int b = gi + BPW * s;
        if (b < KB) {
            int isum, msum;
            float dw, dmw;
            F::dot(r[s], xa[s], c, isum, msum, dw, dmw);
            acc = fmaf(dw * xa[s].d, (float)isum, acc);
            acc = fmaf(-(dmw * xa[s].d), (float)msum, acc);
        }
    }
    if constexpr (RPW == 1) return dpp_wave_sum(acc);
    else return dpp_seg_sum<RPW>(acc);
}

// Row dot product of one weight row (raw registers) with the LDS activation;
// the f32 total is valid in lane 63 (RPW > 1: each 64/RPW-lane segment holds
// its own row, total in the segment's last lane).
template <class F, int SPL, int RPW = 1>
__device__ __forceinline__ float qmv_row(const typename F::Raw (&r)[SPL], const int8_t* s_qs, int qstride,
                                         const float* s_d, const int16_t* s_bs, int gi, int c, int KB) {
    constexpr int BPW = 64 / F::LPB;
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < SPL; s++) {
        const int b = gi + BPW * s;
        if (b < KB) {
            typename F::Act xa;
            F::load_act(s_qs, qstride, s_d, s_bs, b, c, xa);
            int isum, msum;
            float dw, dmw;
            F::dot(r[s], xa, c, isum, msum, dw, dmw);
            acc = fmaf(dw * xa.d, (float)isum, acc);
            acc = fmaf(-(dmw * xa.d), (float)msum, acc);
        }
    }
    if constexpr (RPW == 1) return dpp_wave_sum(acc);
    else return dpp_seg_sum<RPW>(acc);
}

}  // namespace frq
