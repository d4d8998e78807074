// device.h -- gfx950 (CDNA4, wave64) device helpers shared by the kernels of libpurhie_qmv.
//
// Byte layouts are GGUF's (little-endian); see include/quant_types.h for the block maps.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace pq {

constexpr int WAVE = 64;

// fp16 bits -> float (exact)
__device__ __forceinline__ float h2f(uint32_t bits16) { return __half2float(__ushort_as_half((uint16_t)bits16)); }

// Unsigned E4M3 scale byte at half scale, the GGUF ROCmFP4 decoder (reference src/quant_types.cpp:352-357):
// 0x7F..0xFF -> 0, exponent field 0 -> m * 2^-10, else (8 + m) * 2^(E - 11). Built from the exponent bits
// directly: (8 + m) * 2^(E - 11) = 1.m * 2^(E - 8), i.e. float exponent E + 119; subnormals are m * 2^-10.
__device__ __forceinline__ float ue4m3_half(uint32_t e) {
    e &= 0xffu;
    const uint32_t E = e >> 3, m = e & 7u;
    const float normal = __uint_as_float(((E + 119u) << 23) | (m << 20));
    const float sub = (float)m * 0x1p-10f;
    const float v = E == 0 ? sub : normal;
    return e > 0x7eu ? 0.0f : v;
}

// signed int8 dot of 4 bytes, accumulated: v_dot4_i32_i8
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Four 4-bit ROCmFP4 codes (one per byte, 0..15, sign in bit 3) -> four int8 codebook values
// {0, 1, 2, 3, 4, 6, 8, 10} with the sign: two byte lookups (v_perm_b32: positive and negative tables of
// 8) and a byte select by the sign mask. The sign mask is built with v_perm's sign-replicating selectors
// (selector 8..11 = bit 7 of bytes 1, 3, 5, 7 of {S0:S1}) after moving each code's bit 3 to bit 7.
__device__ __forceinline__ int fp4x4(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x0a080604u, 0x03020100u, sel);
    const uint32_t neg = __builtin_amdgcn_perm(0xf6f8fafcu, 0xfdfeff00u, sel);
    const uint32_t s = n << 4;  // bit 3 of byte i -> bit 7 of byte i
    const uint32_t m = __builtin_amdgcn_perm(s, s << 8, 0x0b090a08u);
    return (int)((pos & ~m) | (neg & m));
}

// Four 4-bit codes taken from the high nibbles of the bytes of w
__device__ __forceinline__ int fp4x4_hi(uint32_t w) {
    const uint32_t sel = (w >> 4) & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x0a080604u, 0x03020100u, sel);
    const uint32_t neg = __builtin_amdgcn_perm(0xf6f8fafcu, 0xfdfeff00u, sel);
    const uint32_t m = __builtin_amdgcn_perm(w, w << 8, 0x0b090a08u);  // bit 7 of each byte
    return (int)((pos & ~m) | (neg & m));
}

__device__ __forceinline__ int fp4x4_lo(uint32_t w) { return fp4x4(w & 0x0f0f0f0fu); }

// the dword starting `off` bytes (0..3, run-time) into the 8 bytes {hi:lo}
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t off) {
    return __builtin_amdgcn_alignbyte(hi, lo, off);
}

// 4-byte aligned global loads (the compiler merges consecutive ones into dwordx2/x4)
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)p; }

// the same, non-temporal: weights stream past the caches once (the activation stays cached)
__device__ __forceinline__ uint32_t ld32_nt(const uint8_t *p) { return __builtin_nontemporal_load((const uint32_t *)p); }

struct u32x4 {
    uint32_t x, y, z, w;
};
__device__ __forceinline__ u32x4 ld128(const uint8_t *p) {  // 16-byte aligned
    const uint4 v = *(const uint4 *)p;
    return {v.x, v.y, v.z, v.w};
}
typedef uint32_t u32v4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 ld128_nt(const uint8_t *p) {  // 16-byte aligned, non-temporal
    const u32v4 v = __builtin_nontemporal_load((const u32v4 *)p);
    return {v.x, v.y, v.z, v.w};
}

// Q4_K: 6-bit scale and min of sub-block j from the 12 scale bytes held as 3 dwords (bytes 4..15 of
// the block): j < 4: scale = byte j & 63, min = byte j+4 & 63; else scale = (byte j+4 & 15) | (byte j-4
// >> 6) << 4, min = (byte j+4 >> 4) | (byte j >> 6) << 4 (reference src/quant_types.cpp:193-201).
__device__ __forceinline__ uint32_t byte_of(const uint32_t s[3], int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; }
__device__ __forceinline__ void k4_scale_min(const uint32_t s[3], int j, int &sc, int &mn) {
    if (j < 4) {
        sc = (int)(byte_of(s, j) & 63u);
        mn = (int)(byte_of(s, j + 4) & 63u);
    } else {
        sc = (int)((byte_of(s, j + 4) & 15u) | ((byte_of(s, j - 4) >> 6) << 4));
        mn = (int)((byte_of(s, j + 4) >> 4) | ((byte_of(s, j) >> 6) << 4));
    }
}

// butterfly sum over groups of L lanes (L a power of two <= 64), result in every lane of the group
__device__ __forceinline__ float group_sum(float v, int L) {
    for (int off = L >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return v;
}

}  // namespace pq
