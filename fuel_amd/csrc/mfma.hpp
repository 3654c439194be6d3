// Int8 MFMA building blocks shared by the batched QMatMul kernels
// (mmq.hip, mmq_skinny.hip): operand vector types and the byte-plane
// arithmetic that turns k-quant codes and sub-block scales into exact int8
// MFMA operands.
#pragma once

#include "common.hpp"

namespace frq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

// Four nibble bytes (<= 15) times a small factor (<= 7), byte by byte: each
// product is <= 105, so two 16-bit lane multiplies (one full-rate packed
// instruction) produce them without carries between bytes.
__device__ __forceinline__ int bytes_times(uint32_t q, uint32_t f) {
    const u16x2 p = __builtin_bit_cast(u16x2, q) * u16x2{(unsigned short)f, (unsigned short)f};
    return __builtin_bit_cast(int, p);
}

// Four 6-bit codes u (bytes of q, <= 63) -> w = (u - 32) * sc split into the
// byte planes wl = w & 127 and wh = w >> 7.  Each 16-bit lane holds one
// product exactly (|w| <= 4096), so the arithmetic runs two codes per packed
// instruction: even bytes, then odd bytes.
__device__ __forceinline__ void q6_planes(uint32_t q, uint32_t sc16, uint32_t c16, int& wl, int& wh) {
    const u16x2 ev = __builtin_bit_cast(u16x2, q & 0x00ff00ffu);
    const u16x2 od = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, q, 0x0c030c01u));  // bytes 1, 3
    const u16x2 f = __builtin_bit_cast(u16x2, sc16), c = __builtin_bit_cast(u16x2, c16);
    const u16x2 pe = ev * f + c, po = od * f + c;  // (u - 32) * sc mod 2^16
    // interleave the low bytes of the four lanes back into code order
    const uint32_t sel = 0x06020400u;  // [pe.b0, po.b0, pe.b2, po.b2]
    wl = (int)(__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, po), __builtin_bit_cast(uint32_t, pe), sel) &
               0x7f7f7f7fu);
    const i16x2 he = __builtin_bit_cast(i16x2, pe) >> (short)7, ho = __builtin_bit_cast(i16x2, po) >> (short)7;
    wh = (int)__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ho), __builtin_bit_cast(uint32_t, he), sel);
}

}  // namespace frq
