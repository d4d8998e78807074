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

// Four 4-bit FP4 codes -> four int8 codebook values {0, 1, 2, 3, 4, 6, 8, TOP} with the sign in bit 3:
// two byte lookups by the 3-bit magnitude index (v_perm_b32 on a positive and a negative table of 8), then
// a third v_perm picks, per byte, the positive (selector i) or the negative (selector 4 + i) result, the
// selector built from the sign bit. sel: the magnitude indices (bytes 0..7); fsel: that selector, byte i = i,
// plus 4 where the code is negative. TOP 10: ROCmFP4's codebook; TOP 12: E2M1 at half scale (MXFP4, NVFP4).
// fp4_sel makes fsel from the codes shifted so that each sign bit sits at bit 2 of its byte, in one v_and_or_b32
// (the compiler's own form of the mask and the merge took a mask, a shift and an or).
__device__ __forceinline__ uint32_t fp4_sel(uint32_t sh) {
    uint32_t r;
    __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(sh), "s"(0x04040404u), "v"(0x03020100u));  // (one scalar operand: the constant bus)
    return r;
}

template <int TOP = 10>
__device__ __forceinline__ int fp4_pick(uint32_t sel, uint32_t fsel) {
    const uint32_t pos = __builtin_amdgcn_perm(0x00080604u | (uint32_t)TOP << 24, 0x03020100u, sel);
    const uint32_t neg = __builtin_amdgcn_perm(0x00f8fafcu | (uint32_t)(256 - TOP) << 24, 0xfdfeff00u, sel);
    return (int)__builtin_amdgcn_perm(neg, pos, fsel);
}

// the codes in the low nibbles of the bytes of w
template <int TOP = 10>
__device__ __forceinline__ int fp4x4_lo(uint32_t w) {
    return fp4_pick<TOP>(w & 0x07070707u, fp4_sel(w >> 1));
}

// the codes in the high nibbles of the bytes of w
template <int TOP = 10>
__device__ __forceinline__ int fp4x4_hi(uint32_t w) {
    return fp4_pick<TOP>((w >> 4) & 0x07070707u, fp4_sel(w >> 5));
}

// four codes, one per byte (0..15)
template <int TOP = 10>
__device__ __forceinline__ int fp4x4(uint32_t n) { return fp4x4_lo<TOP>(n); }

// the int8 level of one code (0..15)
template <int TOP = 10>
__device__ __forceinline__ int fp4_level(uint32_t nib) { return (int)(int8_t)(fp4x4<TOP>(nib) & 0xffu); }

// MXFP4's E8M0 scale byte at half scale, 2^(e - 128) (reference src/quant_types.cpp:390-395): e = 0, 1 are the
// float subnormals 2^-128, 2^-127, else the exponent field e - 1
__device__ __forceinline__ float e8m0_half(uint32_t e) {
    e &= 0xffu;
    return __uint_as_float(e < 2 ? 0x00200000u << e : (e - 1) << 23);
}

// NVFP4's scale byte: UE4M3 at half scale, the sign bit ignored (reference src/quant_types.cpp:409-416)
__device__ __forceinline__ float nv_scale(uint32_t e) { return ue4m3_half(e & 0x7fu); }

// Four IQ4_NL / IQ4_XS indices (one per byte, 0..15) -> their int8 levels, ggml's kvalues_iq4nl {-127, -104, -83,
// -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113}: the low 3 bits look up both halves of the table with
// v_perm_b32, bit 3 picks the half per byte (as fp4_pick).
__device__ __forceinline__ int iq4nl4(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(0xf6eaddcfu, 0xbfad9881u, sel);  // indices 0..7
    const uint32_t b = __builtin_amdgcn_perm(0x71594535u, 0x26190d01u, sel);  // indices 8..15
    return (int)__builtin_amdgcn_perm(b, a, fp4_sel(n >> 1));
}

// the indices in the low / high nibbles of the bytes of q
__device__ __forceinline__ int iq4nl4_lo(uint32_t q) {
    const uint32_t sel = q & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(0xf6eaddcfu, 0xbfad9881u, sel);
    const uint32_t b = __builtin_amdgcn_perm(0x71594535u, 0x26190d01u, sel);
    return (int)__builtin_amdgcn_perm(b, a, fp4_sel(q >> 1));
}
__device__ __forceinline__ int iq4nl4_hi(uint32_t q) {
    const uint32_t sel = (q >> 4) & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(0xf6eaddcfu, 0xbfad9881u, sel);
    const uint32_t b = __builtin_amdgcn_perm(0x71594535u, 0x26190d01u, sel);
    return (int)__builtin_amdgcn_perm(b, a, fp4_sel(q >> 5));
}

// IQ4_XS sub-block j's scale ls - 32 from scales_h (16 bits) and scales_l (4 bytes as a dword)
__device__ __forceinline__ int iq4xs_scale(uint32_t sh, uint32_t sl, int j) {
    return (int)(((sl >> (4 * j)) & 0xfu) | (((sh >> (2 * j)) & 3u) << 4)) - 32;
}

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

// Cross-lane reductions without an LDS round trip (a ds_bpermute per step costs ~100 cycles of latency). Within
// each 16-lane row, DPP joins lane pairs (quad_perm 1,0,3,2), quad halves (2,3,0,1), quads (row_half_mirror: lane
// i <- 7 - i) and half rows (row_mirror: i <- 15 - i); once the groups below are whole, every lane of a group holds
// the same value, so each step joins a group with its neighbour. Rows meet through scalar reads of lanes 0, 16, 32,
// 48. One order for a given L (a power of two <= 64), the result in every lane of the group; all lanes active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
constexpr int DPP_PAIR = 0xb1, DPP_QHALF = 0x4e, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

__device__ __forceinline__ float group_sum(float v, int L) {
    if (L >= 2) v += dpp_f<DPP_PAIR>(v);
    if (L >= 4) v += dpp_f<DPP_QHALF>(v);
    if (L >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if (L >= 16) v += dpp_f<DPP_MIRROR>(v);
    if (L >= 32) {
        const float a = readlane_f(v, 0) + readlane_f(v, 16), b = readlane_f(v, 32) + readlane_f(v, 48);
        v = L == 64 ? a + b : (threadIdx.x & 32) ? b : a;
    }
    return v;
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ int group_isum(int v, int L) {
    if (L >= 2) v += dpp_i<DPP_PAIR>(v);
    if (L >= 4) v += dpp_i<DPP_QHALF>(v);
    if (L >= 8) v += dpp_i<DPP_HALF_MIRROR>(v);
    if (L >= 16) v += dpp_i<DPP_MIRROR>(v);
    if (L >= 32) {
        const int a = __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16),
                  b = __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
        v = L == 64 ? a + b : (threadIdx.x & 32) ? b : a;
    }
    return v;
}

__device__ __forceinline__ float group_max(float v, int L) {
    if (L >= 2) v = fmaxf(v, dpp_f<DPP_PAIR>(v));
    if (L >= 4) v = fmaxf(v, dpp_f<DPP_QHALF>(v));
    if (L >= 8) v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    if (L >= 16) v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    if (L >= 32) {
        const float a = fmaxf(readlane_f(v, 0), readlane_f(v, 16)), b = fmaxf(readlane_f(v, 32), readlane_f(v, 48));
        v = L == 64 ? fmaxf(a, b) : (threadIdx.x & 32) ? b : a;
    }
    return v;
}

// Row r of a dense launch: its weights and output (token t at out + t * ystride), and the output scale.
// The argument arrays are read with constant indices and selected: a run-time index into a kernel-argument
// array is a memory load, and its wait would also wait for every weight load issued before it.
struct DenseRows {
    const MvArgs &a;
    template <class T>
    __device__ static T pick(int m, T v0, T v1, T v2, T v3) {
        return m == 0 ? v0 : m == 1 ? v1 : m == 2 ? v2 : v3;
    }
    __device__ int mat(int row) const { return (row >= a.bound[0]) + (row >= a.bound[1]) + (row >= a.bound[2]); }
    __device__ int base(int m) const { return pick(m, 0, a.bound[0], a.bound[1], a.bound[2]); }
    __device__ const uint8_t *w(int row) const {
        const int m = mat(row);
        return pick(m, a.W[0], a.W[1], a.W[2], a.W[3]) + (long long)(row - base(m)) * a.row_bytes;
    }
    __device__ void store(int row, int t, float v) const {
        const int m = mat(row);
        float *y = pick(m, a.y[0], a.y[1], a.y[2], a.y[3]);
        const long long ys = pick(m, a.ystride[0], a.ystride[1], a.ystride[2], a.ystride[3]);
        y[(long long)t * ys + (row - base(m))] = v * pick(m, a.osc[0], a.osc[1], a.osc[2], a.osc[3]);
    }
    // the row's value for each of NT tokens (its matrix, output and scale picked once)
    template <int NT>
    __device__ void store_all(int row, const float (&v)[NT]) const {
        const int m = mat(row);
        float *y = pick(m, a.y[0], a.y[1], a.y[2], a.y[3]) + (row - base(m));
        const long long ys = pick(m, a.ystride[0], a.ystride[1], a.ystride[2], a.ystride[3]);
        const float sc = pick(m, a.osc[0], a.osc[1], a.osc[2], a.osc[3]);
#pragma unroll
        for (int t = 0; t < NT; ++t) y[t * ys] = v[t] * sc;
    }
};

// Capture of the integer dots (the test hook of capture mode): put(t, g, v) adds the dot v of scale group g (of
// the lane's unit, or of its row) for token t. NoCap is the production kernels': it compiles to nothing.
struct NoCap {
    __device__ void put(int, int, int) const {}
};
struct DotCap {
    int32_t *p;    // token 0's group 0 (null: this lane captures nothing)
    long long ts;  // per token
    __device__ void put(int t, int g, int v) const {
        if (p) atomicAdd(p + t * ts + g, v);
    }
};

// Rows of one (matrix, slot, token) of an expert-indexed launch
struct IdRows {
    const uint8_t *W;
    long long rb;
    float *y;
    float sc;
    __device__ const uint8_t *w(int row) const { return W + (long long)row * rb; }
    __device__ void store(int row, int, float v) const { y[row] = v * sc; }
    template <int NT>
    __device__ void store_all(int row, const float (&v)[NT]) const {
        static_assert(NT == 1, "one token a slot");
        y[row] = v[0] * sc;
    }
};

// The entry a block of an expert-indexed launch computes. ids mode: grid.y = slot + n_used * matrix, grid.z =
// token t; the expert is ids[t * n_used + slot] (-1: the matrix Wx), the input row t (or t * n_used + slot with
// x_per_slot), the output row t * n_used + slot. Tiles mode (n_tiles set): grid.y = entry i, grid.z = tile k of
// moe_group's expert tiles; false for the blocks past the last entry (uniform over the block).
struct IdEntry {
    int m, e;
    long long in_row, out_row;
};
__device__ __forceinline__ bool id_entry(const MvIdArgs &a, IdEntry &o) {
    if (a.n_tiles) {
        const int i = blockIdx.y, k = blockIdx.z;
        if (k >= *a.n_tiles || i >= a.tile_n[k]) return false;
        const int st = a.tile_start[k] + i;
        o.m = 0;
        o.e = a.tile_e[k];
        o.in_row = a.in_rows[st];
        o.out_row = a.out_rows[st];
        return true;
    }
    o.m = (int)blockIdx.y >= a.n_used ? 1 : 0;
    const int slot = (int)blockIdx.y - o.m * a.n_used, t = blockIdx.z;
    o.e = a.ids[t * a.n_used + slot];
    o.out_row = (long long)t * a.n_used + slot;
    o.in_row = a.x_per_slot ? o.out_row : t;
    return true;
}

// Tile of a dense GEMM grid (token tiles along x, row tiles along y). The hardware deals workgroups to the 8 XCDs
// round robin by linear id; renumbered, XCD c runs a contiguous range of tiles in which `group` token tiles advance
// together over the row tiles, so the workgroups resident on one XCD share a few activation and weight tiles in its
// L2. Only the order changes (a bijection onto the grid): each tile's arithmetic, and so its bits, stay the same.
__device__ inline void xcd_tile(int &tt, int &rt, int group) {
    const int ntt = gridDim.x, nrt = gridDim.y, nwg = ntt * nrt;
    const int L = blockIdx.x + blockIdx.y * ntt, q = nwg >> 3, r = nwg & 7, c = L & 7;
    const int b = c * q + min(c, r) + (L >> 3);
    const int tg = b / (group * nrt), w = b - tg * group * nrt, gn = min(group, ntt - tg * group);
    tt = tg * group + w % gn;
    rt = w / gn;
}

// Token rows of a GEMM tile: dense tiles take rows base .. base + n - 1 of the activation; MoE tiles take their n
// entries' input rows
struct TokMap {
    const int32_t *rows;  // MoE: in_rows + tile_start (null: dense)
    int base, n;
};

}  // namespace pq
