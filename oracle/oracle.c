/* oracle.c -- CPU restatement of the reference's quantized matrix-product path (see oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker of the HIP product, never linked into it. Citations are
 * file:line in the reference tree (aardbeiplantje/PURHIE). Compiled with -ffp-contract=off
 * -fno-fast-math (oracle/Makefile): the encoders' searches compare float sums whose rounding the
 * reference fixes, and no multiply-add may be fused where the reference does not fuse one.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#if defined(__FAST_MATH__)
#error "oracle.c must not be built with fast math"
#endif

static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ================================================================ scalars */

/* IEEE binary32 -> binary16, round to nearest even; NaN -> 0x7E00 with the sign (the reference's
 * qz_fp32_to_fp16, src/quantize.cpp:28-43, gives the same bits for every input). */
uint16_t orc_f32_to_f16(float f) {
    const uint32_t x = fbits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;
    if (ax >= 0x477ff000u) return sign | 0x7c00u;          /* >= 65520: rounds to infinity */
    if (ax >= 0x38800000u) {                                /* normal half (>= 2^-14) */
        const uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u);
        return sign | (uint16_t)((r - 0x38000000u) >> 13);
    }
    const int e = (int)(ax >> 23);
    if (e == 0) return sign;                               /* float subnormals round to zero */
    const int shift = 126 - e;                             /* value = mant * 2^(e-150) = mant >> shift units of 2^-24 */
    if (shift > 24) return sign;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t r = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return sign | (uint16_t)r;
}

/* binary16 -> binary32, exact (src/quant_types.cpp:16-41) */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in float */
        const float v = (float)m * 0x1p-24f;
        return sign ? -v : v;
    }
    if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13));
    return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_f32_to_f16_n(const float *x, uint16_t *h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(x[i]);
}
void orc_f16_to_f32_n(const uint16_t *h, float *x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_f16_to_f32(h[i]);
}

/* Unsigned E4M3 scale byte -> half-scale value (src/quant_types.cpp:352-357): bytes 0x7F..0xFF are 0,
 * exponent field 0 is subnormal m * 2^-10, else (8 + m) * 2^(E - 11). */
float orc_ue4m3_half(uint8_t e) {
    if (e > 0x7e) return 0.0f;
    const int E = e >> 3, m = e & 7;
    return E == 0 ? ldexpf((float)m, -10) : ldexpf((float)(8 + m), E - 11);
}

/* The legacy decoder of src/fp4_common.h:59-70 (gemm_act_fp4 only): exponent field bits 3..6 (bit 7
 * ignored), subnormal m * 2^-9, normal (1 + m/8) * 2^(E - 8), then halved. */
float orc_ue4m3_fp4common(uint8_t e) {
    const int E = (e >> 3) & 0xf, m = e & 7;
    const float raw = E == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), E - 11);
    return raw * 0.5f;
}

/* Signed FP4 codebook at half scale, sign in bit 3 (src/quant_types.cpp:349) */
static const int8_t k_cb[16] = {0, 1, 2, 3, 4, 6, 8, 10, 0, -1, -2, -3, -4, -6, -8, -10};

/* E2M1 at half scale, MXFP4's and NVFP4's codebook (src/quant_types.cpp:387): the same magnitudes with 12 on
 * top (E2M1's 6 doubled) */
static const int8_t k_e2m1[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* E8M0 exponent byte -> 2^(e - 128), the half-scale value (src/quant_types.cpp:390-395): e = 0, 1 are the
 * subnormals 2^-128, 2^-127 */
float orc_e8m0_half(uint8_t e) { return ldexpf(1.0f, (int)e - 128); }

/* NVFP4's scale byte: UE4M3 at half scale with the sign bit cleared (src/quant_types.cpp:409-416) */
static inline float nv_scale(uint8_t e) { return orc_ue4m3_half((uint8_t)(e & 0x7f)); }

static inline float rd16(const uint8_t *p) { uint16_t h; memcpy(&h, p, 2); return orc_f16_to_f32(h); }

/* ================================================================ formats */

int orc_block_size(int t) {
    switch (t) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q8_0: case ORC_FP4: case ORC_FAST: case ORC_MXFP4: return 32;
    case ORC_NVFP4: return 64;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_IQ4_XS: return 256;
    default: return 0;
    }
}

int orc_type_size(int t) {
    switch (t) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q8_0: return 34;
    case ORC_FP4: return 18;
    case ORC_FAST: case ORC_MXFP4: return 17;
    case ORC_NVFP4: return 36;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_IQ4_XS: return 136;
    default: return 0;
    }
}

size_t orc_row_size(int t, int64_t k) {
    const int b = orc_block_size(t);
    if (!b || k % b) return 0;
    return (size_t)(k / b) * (size_t)orc_type_size(t);
}

/* 6-bit scale / min j of a Q4_K super-block from its 12 packed bytes (src/quant_types.cpp:193-201) */
static inline void k4_scale_min(int j, const uint8_t *q, int *sc, int *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Q4_K level of value v (0..255) of a super-block: chunk v/64, low nibble for the first 32 of the chunk */
static inline int k4_level(const uint8_t *blk, int v) {
    const uint8_t b = blk[16 + 32 * (v >> 6) + (v & 31)];
    return (v & 32) ? (b >> 4) : (b & 0xf);
}

/* Q5_K level (0..31) of value v of a super-block (src/quant_types.cpp:290-314): Q4_K's nibble from ql (bytes
 * 48..175) plus bit 2c (low nibble) or 2c + 1 (high nibble) of qh byte v % 32 (bytes 16..47) as bit 4 */
static inline int k5_level(const uint8_t *blk, int v) {
    const int c = v >> 6, hi = (v >> 5) & 1, l = v & 31;
    const uint8_t b = blk[48 + 32 * c + l];
    return (hi ? (b >> 4) : (b & 0xf)) | (((blk[16 + l] >> (2 * c + hi)) & 1) << 4);
}

/* IQ4_XS (src/quant_types.cpp:111-125): ggml's non-linear 4-bit levels, a nibble indexing kvalues_iq4nl;
 * super-block d (fp16 @0), the 6-bit sub-block scales as scales_h (2 bits each, u16 @2) and scales_l (4 bits,
 * two a byte, @4), qs[128] @8: sub-block j's bytes 8 + 16 j .. + 15 hold values 32 j + i (low nibble) and
 * 32 j + 16 + i (high nibble) */
static const int8_t k_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
static inline int iq4xs_scale(const uint8_t *blk, int j) {  /* ls - 32, in -32 .. 31 */
    const int sh = blk[2] | (blk[3] << 8);
    return (((blk[4 + j / 2] >> (4 * (j & 1))) & 0xf) | (((sh >> (2 * j)) & 3) << 4)) - 32;
}
static inline int iq4xs_level(const uint8_t *blk, int v) {  /* the codebook value of value v (0..255) */
    const int j = v >> 5, i = v & 31;
    const uint8_t b = blk[8 + 16 * j + (i & 15)];
    return k_iq4nl[i < 16 ? (b & 0xf) : (b >> 4)];
}

/* Q6_K raw level (0..63) of value v of a super-block (src/quant_types.cpp:319-344): half h = v/128,
 * within it quarter j = (v%128)/32 and l = v%32; ql byte l (+32 for odd j), high nibble for j >= 2;
 * qh byte l, bits 2j. */
static inline int k6_level(const uint8_t *blk, int v) {
    const int h = v >> 7, j = (v >> 5) & 3, l = v & 31;
    const uint8_t ql = blk[64 * h + l + 32 * (j & 1)];
    const uint8_t qh = blk[128 + 32 * h + l];
    const int lo = (j >= 2) ? (ql >> 4) : (ql & 0xf);
    return lo | (((qh >> (2 * j)) & 3) << 4);
}

/* Decoders: src/quant_types.cpp:182-189 (Q8_0), 193-201/265-287 (Q4_K), 319-344 (Q6_K), 359-382 (FP4, FAST) */
int orc_to_float(int t, const void *src, float *y, int64_t n) {
    const int bs = orc_block_size(t);
    if (!bs || n % bs) return -1;
    const uint8_t *b = (const uint8_t *)src;
    switch (t) {
    case ORC_F32: memcpy(y, src, (size_t)n * 4); return 0;
    case ORC_F16: for (int64_t i = 0; i < n; ++i) y[i] = rd16(b + 2 * i); return 0;
    case ORC_BF16:
        for (int64_t i = 0; i < n; ++i) { uint16_t h; memcpy(&h, b + 2 * i, 2); y[i] = bitsf((uint32_t)h << 16); }
        return 0;
    case ORC_Q8_0:
        for (int64_t i = 0; i < n / 32; ++i, b += 34, y += 32) {
            const float d = rd16(b);
            for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
        }
        return 0;
    case ORC_Q4_K:
        for (int64_t i = 0; i < n / 256; ++i, b += 144) {
            const float d = rd16(b), dmin = rd16(b + 2);
            for (int c = 0; c < 4; ++c) {
                int sc, mn;
                k4_scale_min(2 * c, b + 4, &sc, &mn);
                const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                k4_scale_min(2 * c + 1, b + 4, &sc, &mn);
                const float d2 = d * (float)sc, m2 = dmin * (float)mn;
                for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(b[16 + 32 * c + l] & 0xf) - m1;
                for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(b[16 + 32 * c + l] >> 4) - m2;
            }
        }
        return 0;
    case ORC_Q5_K:
        for (int64_t i = 0; i < n / 256; ++i, b += 176) {
            const float d = rd16(b), dmin = rd16(b + 2);
            for (int c = 0; c < 4; ++c) {
                int sc, mn;
                k4_scale_min(2 * c, b + 4, &sc, &mn);
                const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                k4_scale_min(2 * c + 1, b + 4, &sc, &mn);
                const float d2 = d * (float)sc, m2 = dmin * (float)mn;
                for (int l = 0; l < 32; ++l) *y++ = d1 * (float)k5_level(b, 64 * c + l) - m1;
                for (int l = 0; l < 32; ++l) *y++ = d2 * (float)k5_level(b, 64 * c + 32 + l) - m2;
            }
        }
        return 0;
    case ORC_Q6_K:
        for (int64_t i = 0; i < n / 256; ++i, b += 210, y += 256) {
            const float d = rd16(b + 208);
            const int8_t *sc = (const int8_t *)(b + 192);
            for (int v = 0; v < 256; ++v) {
                const int q = k6_level(b, v) - 32;
                y[v] = d * (float)sc[v >> 4] * (float)q;   /* (d * sc) * q, src/quant_types.cpp:337-340 */
            }
        }
        return 0;
    case ORC_IQ4_XS:
        for (int64_t i = 0; i < n / 256; ++i, b += 136, y += 256) {
            const float d = rd16(b);
            for (int v = 0; v < 256; ++v) {
                const float dl = d * (float)iq4xs_scale(b, v >> 5);   /* d * (ls - 32), then * value */
                y[v] = dl * (float)iq4xs_level(b, v);
            }
        }
        return 0;
    case ORC_FP4:
        for (int64_t i = 0; i < n / 32; ++i, b += 18, y += 32) {
            const float d0 = orc_ue4m3_half(b[16]), d1 = orc_ue4m3_half(b[17]);
            for (int j = 0; j < 16; ++j) {
                y[j] = (float)k_cb[b[j] & 0xf] * d0;
                y[j + 16] = (float)k_cb[b[j] >> 4] * d1;
            }
        }
        return 0;
    case ORC_FAST:
        for (int64_t i = 0; i < n / 32; ++i, b += 17, y += 32) {
            const float d = orc_ue4m3_half(b[16]);
            for (int j = 0; j < 16; ++j) {
                y[j] = (float)k_cb[b[j] & 0xf] * d;
                y[j + 16] = (float)k_cb[b[j] >> 4] * d;
            }
        }
        return 0;
    case ORC_MXFP4:   /* e, then the FAST value bytes (src/quant_types.cpp:397-407) */
        for (int64_t i = 0; i < n / 32; ++i, b += 17, y += 32) {
            const float d = orc_e8m0_half(b[0]);
            for (int j = 0; j < 16; ++j) {
                y[j] = (float)k_e2m1[b[1 + j] & 0xf] * d;
                y[j + 16] = (float)k_e2m1[b[1 + j] >> 4] * d;
            }
        }
        return 0;
    case ORC_NVFP4:   /* four scales, then four 8-byte sub-blocks of 16 values (src/quant_types.cpp:409-422) */
        for (int64_t i = 0; i < n / 64; ++i, b += 36) {
            for (int s = 0; s < 4; ++s, y += 16) {
                const float d = nv_scale(b[s]);
                for (int j = 0; j < 8; ++j) {
                    y[j] = (float)k_e2m1[b[4 + 8 * s + j] & 0xf] * d;
                    y[j + 8] = (float)k_e2m1[b[4 + 8 * s + j] >> 4] * d;
                }
            }
        }
        return 0;
    }
    return -1;
}

/* ================================================================ encoders */

/* ggml's nearest_int: round half to even by adding 1.5 * 2^23 (src/quantize.cpp:161-167). Valid for
 * |v| < 2^22, the range every caller stays in. */
static inline int nint(float v) {
    const float s = v + 12582912.f;
    int32_t i;
    memcpy(&i, &s, 4);
    return (i & 0x007fffff) - 0x00400000;
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* Q8_0 weights (src/quantize.cpp:53-64): amax with ggml's MAX (a NaN wins), d = amax / 127 stored as fp16,
 * q = roundf(x / d) via the reciprocal, half away from zero. */
static void enc_q8_0(const float *x, uint8_t *out, int64_t k) {
    for (int64_t i = 0; i < k / 32; ++i, x += 32, out += 34) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(x[j]);
            amax = amax > a ? amax : a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t h = orc_f32_to_f16(d);
        memcpy(out, &h, 2);
        for (int j = 0; j < 32; ++j) out[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    }
}

/* ggml's make_qkx2_quants (src/quantize.cpp:169-244): an asymmetric scale / min search over nstep
 * candidate inverse scales, weighted least squares, keeping the best error strictly. Returns the
 * scale; *neg_min receives -min. */
static float qkx2(int n, int nmax, const float *x, const float *w, uint8_t *L, float *neg_min, uint8_t *Laux,
                  float rmin, float rdelta, int nstep) {
    float lo = x[0], hi = x[0];
    float sw = w[0];
    float sx = sw * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sw += w[i];
        sx += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        memset(L, 0, (size_t)n);
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = (float)nmax / (hi - lo);
    float scale = 1.0f / iscale;
    float best = 0.0f;
    for (int i = 0; i < n; ++i) {
        const int l = clampi(nint(iscale * (x[i] - lo)), 0, nmax);
        L[i] = (uint8_t)l;
        const float diff = scale * (float)L[i] + lo - x[i];
        best += w[i] * (diff * diff);
    }
    if (nstep < 1) {
        *neg_min = -lo;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < n; ++i) {
            const int l = clampi(nint(iscale * (x[i] - lo)), 0, nmax);
            Laux[i] = (uint8_t)l;
            sl += w[i] * (float)l;
            sl2 += w[i] * (float)l * (float)l;
            sxl += w[i] * (float)l * x[i];
        }
        const float D = sw * sl2 - sl * sl;
        if (D > 0) {
            float ts = (sw * sxl - sx * sl) / D;
            float tm = (sl2 * sx - sl * sxl) / D;
            if (tm > 0) {
                tm = 0;
                ts = sxl / sl2;
            }
            float cur = 0;
            for (int i = 0; i < n; ++i) {
                const float diff = ts * (float)Laux[i] + tm - x[i];
                cur += w[i] * (diff * diff);
            }
            if (cur < best) {
                memcpy(L, Laux, (size_t)n);
                best = cur;
                scale = ts;
                lo = tm;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

/* The K-quant super-block of Q4_K / Q5_K (src/quantize.cpp:246-307, kq_super_block): eight sub-block searches
 * (weights av_x + |x|; Q4_K nmax 15, rmin -1, 20 steps; Q5_K nmax 31, rmin -0.5, 15 steps), 6-bit scales / mins
 * relative to the largest packed into 12 bytes, fp16 d = max_scale / 63 and dmin = max_min / 63, then the levels
 * re-derived from the packed scales, clamped to [0, nmax]. */
static void kq_block(const float *x, int nmax, float rmin, int nstep, uint8_t *L, uint8_t *scl, uint16_t *hd,
                     uint16_t *hm) {
    uint8_t Laux[32];
    float w[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float s2 = 0;
        for (int l = 0; l < 32; ++l) s2 += x[32 * j + l] * x[32 * j + l];
        const float av = sqrtf(s2 / 32);
        for (int l = 0; l < 32; ++l) w[l] = av + fabsf(x[32 * j + l]);
        scales[j] = qkx2(32, nmax, x + 32 * j, w, L + 32 * j, &mins[j], Laux, rmin, 0.1f, nstep);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_s = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_m = max_min > 0 ? 63.f / max_min : 0.f;
    memset(scl, 0, 12);
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)nint(inv_s * scales[j]);
        uint8_t lm = (uint8_t)nint(inv_m * mins[j]);
        if (ls > 63) ls = 63;
        if (lm > 63) lm = 63;
        if (j < 4) {
            scl[j] = ls;
            scl[j + 4] = lm;
        } else {
            scl[j + 4] = (uint8_t)((ls & 0xf) | ((lm & 0xf) << 4));
            scl[j - 4] |= (uint8_t)((ls >> 4) << 6);
            scl[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    *hd = orc_f32_to_f16(max_scale / 63.f);
    *hm = orc_f32_to_f16(max_min / 63.f);
    const float fd = orc_f16_to_f32(*hd), fm = orc_f16_to_f32(*hm);
    for (int j = 0; j < 8; ++j) {
        int sc, mn;
        k4_scale_min(j, scl, &sc, &mn);
        const float d = fd * (float)sc;
        if (d == 0.0f) continue;
        const float dm = fm * (float)mn;
        for (int i = 0; i < 32; ++i) L[32 * j + i] = (uint8_t)clampi(nint((x[32 * j + i] + dm) / d), 0, nmax);
    }
}

/* Q4_K (src/quantize.cpp:309-325): d, dmin, scales, then chunk c's 32 bytes hold values 64 c + l (low nibble)
 * and 64 c + 32 + l (high nibble) */
static void enc_q4_k(const float *x, uint8_t *out, int64_t k) {
    for (int64_t b = 0; b < k / 256; ++b, x += 256, out += 144) {
        uint8_t L[256];
        uint16_t hd, hm;
        kq_block(x, 15, -1.0f, 20, L, out + 4, &hd, &hm);
        memcpy(out, &hd, 2);
        memcpy(out + 2, &hm, 2);
        uint8_t *q = out + 16;
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l) q[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
    }
}

/* Q5_K (src/quantize.cpp:327-358): as Q4_K with 5-bit levels; the low 4 bits as Q4_K's nibbles (ql, bytes
 * 48..175), bit 4 of value 64 c + l in qh byte l bit 2 c, of value 64 c + 32 + l in bit 2 c + 1 (bytes 16..47) */
static void enc_q5_k(const float *x, uint8_t *out, int64_t k) {
    for (int64_t b = 0; b < k / 256; ++b, x += 256, out += 176) {
        uint8_t L[256];
        uint16_t hd, hm;
        kq_block(x, 31, -0.5f, 15, L, out + 4, &hd, &hm);
        memcpy(out, &hd, 2);
        memcpy(out + 2, &hm, 2);
        uint8_t *qh = out + 16, *ql = out + 48;
        memset(qh, 0, 32);
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l) {
                const int l1 = L[64 * c + l], l2 = L[64 * c + 32 + l];
                qh[l] |= (uint8_t)(((l1 >> 4) << (2 * c)) | ((l2 >> 4) << (2 * c + 1)));
                ql[32 * c + l] = (uint8_t)((l1 & 0xf) | ((l2 & 0xf) << 4));
            }
    }
}

/* ggml's make_qx_quants with rmse_type 1 and no importance (src/quantize.cpp:330-396): a symmetric scale
 * from the signed value of largest magnitude, refined over 18 candidate inverse scales, weights x^2. L
 * receives levels + nmax. */
static float qx(int n, int nmax, const float *x, int8_t *L) {
    float mx = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) {
            amax = a;
            mx = x[i];
        }
    }
    if (amax < 1e-15f) {
        memset(L, 0, (size_t)n);
        return 0.0f;
    }
    float iscale = (float)(-nmax) / mx;
    float slx = 0, sl2 = 0;
    for (int i = 0; i < n; ++i) {
        const int l = clampi(nint(iscale * x[i]), -nmax, nmax - 1);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        slx += w * x[i] * (float)l;
        sl2 += w * (float)l * (float)l;
    }
    float scale = sl2 != 0.0f ? slx / sl2 : 0.0f;
    float best = scale * slx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / mx;
        slx = sl2 = 0;
        for (int i = 0; i < n; ++i) {
            const int l = clampi(nint(iscale * x[i]), -nmax, nmax - 1);
            const float w = x[i] * x[i];
            slx += w * x[i] * (float)l;
            sl2 += w * (float)l * (float)l;
        }
        if (sl2 > 0 && slx * slx > best * sl2) {
            for (int i = 0; i < n; ++i) L[i] = (int8_t)(nmax + clampi(nint(iscale * x[i]), -nmax, nmax - 1));
            scale = slx / sl2;
            best = scale * slx;
        }
    }
    return scale;
}

/* Q6_K (src/quantize.cpp:398-444): sixteen 16-value searches, int8 scales relative to the largest
 * (iscale -128 / max_scale), fp16 d = 1 / iscale, levels re-derived from the rounded scales. */
static void enc_q6_k(const float *x, uint8_t *out, int64_t k) {
    for (int64_t b = 0; b < k / 256; ++b, x += 256, out += 210) {
        int8_t L[256];
        float scales[16];
        float max_scale = 0, max_abs = 0;
        for (int g = 0; g < 16; ++g) {
            const float s = qx(16, 32, x + 16 * g, L + 16 * g);
            scales[g] = s;
            if (fabsf(s) > max_abs) {
                max_abs = fabsf(s);
                max_scale = s;
            }
        }
        memset(out, 0, 210);
        if (max_abs < 1e-15f) continue;
        const float iscale = -128.f / max_scale;
        const uint16_t hd = orc_f32_to_f16(1.0f / iscale);
        memcpy(out + 208, &hd, 2);
        int8_t *sc = (int8_t *)(out + 192);
        for (int g = 0; g < 16; ++g) {
            const int v = nint(iscale * scales[g]);
            sc[g] = (int8_t)(v < 127 ? v : 127);
        }
        const float fd = orc_f16_to_f32(hd);
        for (int g = 0; g < 16; ++g) {
            const float d = fd * (float)sc[g];
            if (d == 0.0f) continue;
            for (int i = 0; i < 16; ++i) L[16 * g + i] = (int8_t)(clampi(nint(x[16 * g + i] / d), -32, 31) + 32);
        }
        uint8_t *ql = out, *qh = out + 128;
        for (int h = 0; h < 2; ++h) {
            const int8_t *Lh = L + 128 * h;
            for (int l = 0; l < 32; ++l) {
                ql[l] = (uint8_t)((Lh[l] & 0xf) | ((Lh[l + 64] & 0xf) << 4));
                ql[l + 32] = (uint8_t)((Lh[l + 32] & 0xf) | ((Lh[l + 96] & 0xf) << 4));
                qh[l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) |
                                  ((Lh[l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
    }
}

/* ROCmFP4 scale search (src/quantize.cpp:946-1109, ROCmFPX rocmfp4.c without an importance matrix) */
static float g_half[127];
static pthread_once_t g_half_once = PTHREAD_ONCE_INIT;
static void half_init(void) {
    for (int e = 0; e < 127; ++e) g_half[e] = orc_ue4m3_half((uint8_t)e);
}
static inline float shalf(int e) { return e <= 0x7e ? g_half[e] : 0.0f; }

/* codebook magnitude index of |x * inv|: ties to the lower magnitude (<= at each midpoint) */
static inline int mag_index(float a) {
    if (a <= 0.5f) return 0;
    if (a <= 1.5f) return 1;
    if (a <= 2.5f) return 2;
    if (a <= 3.5f) return 3;
    if (a <= 5.0f) return 4;
    if (a <= 7.0f) return 5;
    if (a <= 9.0f) return 6;
    return 7;
}
static const float k_mag[8] = {0, 1, 2, 3, 4, 6, 8, 10};

static inline uint8_t fp4_code(float x, float inv) {
    if (!isfinite(x)) return 0;
    const int m = mag_index(fabsf(x * inv));
    if (m == 0) return 0;
    return (uint8_t)(x < 0.0f ? (m | 8) : m);
}

static inline float fp4_decoded(float x, float inv) {
    if (!isfinite(x)) return 0.0f;
    const float m = k_mag[mag_index(fabsf(x * inv))];
    return x < 0.0f ? -m : m;
}

/* squared error of n values at scale byte e, abandoned (returning a value > cap) once above cap */
static float fp4_err(const float *x, int n, int e, float cap) {
    const float s = shalf(e);
    const float inv = 1.0f / s;
    float err = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float y = fp4_decoded(x[i], inv) * s;
        const float d = x[i] - y;
        err += d * d;
        if (err > cap) return err;
    }
    return err;
}

/* the byte in 1..126 whose scale is nearest target, the lower on a midpoint tie */
static int fp4_nearest(float target) {
    if (!(target > 0.0f) || !isfinite(target)) return 1;
    int lo = 1, hi = 126;
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (shalf(mid) < target) lo = mid + 1;
        else hi = mid;
    }
    if (lo == 1) return 1;
    const float up = shalf(lo), dn = shalf(lo - 1);
    return (target - dn <= up - target) ? lo - 1 : lo;
}

/* exhaustive least-squares search outward from the scale nearest max|x| / 10; the lower byte wins a tie;
 * the downward side stops once clipping the largest value alone costs more than the best error */
static uint8_t fp4_scale(const float *x, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    if (!(amax > 0.0f) || !isfinite(amax)) return 0;
    const int start = fp4_nearest(amax / 10.0f);
    int best_e = 0;
    float best = FLT_MAX;
    int down_done = 0;
    for (int delta = 0; delta <= 125; ++delta) {
        const int e0 = start - delta;
        if (!down_done && e0 >= 1 && e0 <= 126) {
            const float clip = amax - 10.0f * shalf(e0);
            if (clip > 0.0f && clip * clip > best) {
                down_done = 1;
            } else {
                const float err = fp4_err(x, n, e0, best);
                if (err < best || (err == best && e0 < best_e)) { best = err; best_e = e0; }
            }
        }
        const int e1 = start + delta;
        if (delta != 0 && e1 >= 1 && e1 <= 126) {
            const float err = fp4_err(x, n, e1, best);
            if (err < best || (err == best && e1 < best_e)) { best = err; best_e = e1; }
        }
        if ((down_done || e0 <= 1) && e1 >= 126) break;
    }
    return (uint8_t)best_e;
}

static inline float fp4_inv(uint8_t e) {
    const float s = shalf(e);
    return s > 0.0f ? 1.0f / s : 0.0f;
}

static void enc_fp4(const float *x, uint8_t *out, int64_t k) {
    for (int64_t i = 0; i < k / 32; ++i, x += 32, out += 18) {
        const uint8_t e0 = fp4_scale(x, 16), e1 = fp4_scale(x + 16, 16);
        const float i0 = fp4_inv(e0), i1 = fp4_inv(e1);
        for (int j = 0; j < 16; ++j) out[j] = (uint8_t)(fp4_code(x[j], i0) | (fp4_code(x[j + 16], i1) << 4));
        out[16] = e0;
        out[17] = e1;
    }
}

static void enc_fast(const float *x, uint8_t *out, int64_t k) {
    for (int64_t i = 0; i < k / 32; ++i, x += 32, out += 17) {
        const uint8_t e = fp4_scale(x, 32);
        const float inv = fp4_inv(e);
        for (int j = 0; j < 16; ++j) out[j] = (uint8_t)(fp4_code(x[j], inv) | (fp4_code(x[j + 16], inv) << 4));
        out[16] = e;
    }
}

/* ggml's best_index_int8 over the sorted codebook: the nearest value, the lower one on a tie
 * (src/quantize.cpp:838-849) */
static int iq4_index(float x) {
    if (x <= k_iq4nl[0]) return 0;
    if (x >= k_iq4nl[15]) return 15;
    int lo = 0, hi = 15;
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (x < k_iq4nl[mid]) hi = mid;
        else lo = mid;
    }
    return x - k_iq4nl[hi - 1] < k_iq4nl[hi] - x ? hi - 1 : hi;
}

/* IQ4_XS (src/quantize.cpp:851-958, 960-974; ggml's quantize_row_iq4_nl_impl without importance weights, 7
 * retries): per 32-value sub-block, weights x^2, a first scale from the signed largest value (d = -max / -127),
 * the least-squares scale of its levels, then 15 candidate inverse scales (itry - 127) / max, keeping the one
 * whose sumqx^2 / sumq2 is largest; the sub-block scales are quantized to 6 bits against d = -max_scale / 32 (the
 * fp32 d, not its fp16 rounding) and each value re-indexed with its sub-block's d * l */
static void enc_iq4_xs(const float *x, uint8_t *out, int64_t k) {
    for (int64_t b = 0; b < k / 256; ++b, x += 256, out += 136) {
        uint8_t L[256];
        float scales[8];
        float max_scale = 0, amax_scale = 0;
        memset(L, 0, sizeof L);
        for (int ib = 0; ib < 8; ++ib) {
            const float *xb = x + 32 * ib;
            float w[32];
            for (int j = 0; j < 32; ++j) w[j] = xb[j] * xb[j];
            float amax = 0, mx = 0;
            for (int j = 0; j < 32; ++j) {
                const float ax = fabsf(xb[j]);
                if (ax > amax) {
                    amax = ax;
                    mx = xb[j];
                }
            }
            if (amax < 1e-15f) {
                scales[ib] = 0;
                continue;
            }
            float d = -mx / (float)k_iq4nl[0];
            float id = 1 / d;
            float sumqx = 0, sumq2 = 0;
            for (int j = 0; j < 32; ++j) {
                const int l = iq4_index(id * xb[j]);
                L[32 * ib + j] = (uint8_t)l;
                const float q = (float)k_iq4nl[l];
                sumqx += w[j] * q * xb[j];
                sumq2 += w[j] * q * q;
            }
            d = sumq2 > 0 ? sumqx / sumq2 : 0.f;
            float best = d * sumqx;
            for (int itry = -7; itry <= 7; ++itry) {
                id = ((float)itry + (float)k_iq4nl[0]) / mx;
                sumqx = sumq2 = 0;
                for (int j = 0; j < 32; ++j) {
                    const int l = iq4_index(id * xb[j]);
                    const float q = (float)k_iq4nl[l];
                    sumqx += w[j] * q * xb[j];
                    sumq2 += w[j] * q * q;
                }
                if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                    d = sumqx / sumq2;
                    best = d * sumqx;
                }
            }
            scales[ib] = d;
            if (fabsf(d) > amax_scale) {
                amax_scale = fabsf(d);
                max_scale = d;
            }
        }
        const float d = -max_scale / 32;
        const uint16_t dh = orc_f32_to_f16(d);
        const float id = d != 0.0f ? 1 / d : 0.f;
        uint16_t sh = 0;
        uint8_t sl[4] = {0, 0, 0, 0};
        for (int ib = 0; ib < 8; ++ib) {
            int l = nint(id * scales[ib]);
            l = l < -32 ? -32 : l > 31 ? 31 : l;
            const float dl = d * (float)l;
            const float idl = dl != 0.0f ? 1 / dl : 0.f;
            for (int j = 0; j < 32; ++j) L[32 * ib + j] = (uint8_t)iq4_index(idl * x[32 * ib + j]);
            l += 32;
            if (ib % 2 == 0) sl[ib / 2] = (uint8_t)(l & 0xf);
            else sl[ib / 2] |= (uint8_t)((l & 0xf) << 4);
            sh |= (uint16_t)((l >> 4) << (2 * ib));
        }
        memcpy(out, &dh, 2);
        memcpy(out + 2, &sh, 2);
        memcpy(out + 4, sl, 4);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 16; ++j) out[8 + 16 * i + j] = (uint8_t)(L[32 * i + j] | (L[32 * i + 16 + j] << 4));
    }
}

/* ggml's best_index_mxfp4: the codebook entry whose value times e is nearest x, the first on a tie
 * (src/quantize.cpp:697-709) */
static uint8_t e2m1_index(float x, float e) {
    int best = 0;
    float best_err = fabsf((float)k_e2m1[0] * e - x);
    for (int i = 1; i < 16; ++i) {
        const float err = fabsf((float)k_e2m1[i] * e - x);
        if (err < best_err) { best = i; best_err = err; }
    }
    return (uint8_t)best;
}

/* MXFP4 (src/quantize.cpp:711-729): e = floor(log2(amax)) - 2 + 127 (log2f; the float converted as the
 * reference's x86 build does, through int32), d = 2^(e - 128), each value's nearest E2M1 level */
static void enc_mxfp4(const float *x, uint8_t *out, int64_t k) {
    for (int64_t i = 0; i < k / 32; ++i, x += 32, out += 17) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j)
            if (amax < fabsf(x[j])) amax = fabsf(x[j]);
        const uint8_t e = amax > 0.0f ? (uint8_t)(int32_t)(floorf(log2f(amax)) - 2 + 127) : 0;
        const float d = orc_e8m0_half(e);
        out[0] = e;
        for (int j = 0; j < 16; ++j) out[1 + j] = (uint8_t)(e2m1_index(x[j], d) | (e2m1_index(x[16 + j], d) << 4));
    }
}

/* ggml_fp32_to_ue4m3 (src/quantize.cpp:670-694): round to nearest on the fp32 bits (the bit below the 3
 * mantissa bits decides), clamped to 448 and the largest code 0x7E, subnormals m * 2^-9 by x * 512 + 0.5 */
static uint8_t f32_to_ue4m3(float x) {
    if (!(x > 0.0f)) return 0;
    if (x > 448.0f) x = 448.0f;
    uint32_t bits;
    memcpy(&bits, &x, 4);
    int e = (int)((bits >> 23) & 0xff) - 127 + 7;
    if (e <= 0) {
        int m = (int)(x * 512.0f + 0.5f);
        if (m > 7) m = 7;
        return m < 1 ? 0 : (uint8_t)m;
    }
    if (e >= 15) return 0x7e;
    int m = (int)((bits >> 20) & 7) + (int)((bits >> 19) & 1);
    if (m > 7) {
        m = 0;
        if (++e >= 15) return 0x7e;
    }
    return (uint8_t)((e << 3) | m);
}

/* NVFP4 (src/quantize.cpp:731-750): per 16 values the UE4M3 code of amax / 6, its half-scale value d, each
 * value's nearest E2M1 level */
static void enc_nvfp4(const float *x, uint8_t *out, int64_t k) {
    for (int64_t i = 0; i < k / 64; ++i, x += 64, out += 36) {
        for (int s = 0; s < 4; ++s) {
            const float *xb = x + 16 * s;
            float amax = 0.0f;
            for (int j = 0; j < 16; ++j)
                if (amax < fabsf(xb[j])) amax = fabsf(xb[j]);
            const uint8_t ue = f32_to_ue4m3(amax / 6.0f);
            const float d = orc_ue4m3_half(ue);
            out[s] = ue;
            for (int j = 0; j < 8; ++j)
                out[4 + 8 * s + j] = (uint8_t)(e2m1_index(xb[j], d) | (e2m1_index(xb[8 + j], d) << 4));
        }
    }
}

static void enc_row(int t, const float *x, uint8_t *y, int64_t k) {
    switch (t) {
    case ORC_F32: memcpy(y, x, (size_t)k * 4); break;
    case ORC_F16: for (int64_t i = 0; i < k; ++i) { const uint16_t h = orc_f32_to_f16(x[i]); memcpy(y + 2 * i, &h, 2); } break;
    case ORC_Q8_0: enc_q8_0(x, y, k); break;
    case ORC_Q4_K: enc_q4_k(x, y, k); break;
    case ORC_Q5_K: enc_q5_k(x, y, k); break;
    case ORC_IQ4_XS: enc_iq4_xs(x, y, k); break;
    case ORC_Q6_K: enc_q6_k(x, y, k); break;
    case ORC_FP4: enc_fp4(x, y, k); break;
    case ORC_FAST: enc_fast(x, y, k); break;
    case ORC_MXFP4: enc_mxfp4(x, y, k); break;
    case ORC_NVFP4: enc_nvfp4(x, y, k); break;
    }
}

/* ---- a minimal row-parallel driver (pthreads, rows split into contiguous chunks) */
typedef struct {
    void (*fn)(void *ctx, int64_t r0, int64_t r1);
    void *ctx;
    int64_t r0, r1;
} span_t;

static void *span_run(void *p) {
    span_t *s = (span_t *)p;
    s->fn(s->ctx, s->r0, s->r1);
    return NULL;
}

static int ncores(void) {
    const long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

static void par_rows(int64_t nrows, int n_threads, void (*fn)(void *, int64_t, int64_t), void *ctx) {
    if (n_threads <= 0) n_threads = ncores();
    if (n_threads > 256) n_threads = 256;
    if (n_threads > nrows) n_threads = nrows > 0 ? (int)nrows : 1;
    if (n_threads <= 1) {
        fn(ctx, 0, nrows);
        return;
    }
    pthread_t th[256];
    span_t sp[256];
    for (int i = 0; i < n_threads; ++i) {
        sp[i].fn = fn;
        sp[i].ctx = ctx;
        sp[i].r0 = nrows * i / n_threads;
        sp[i].r1 = nrows * (i + 1) / n_threads;
        pthread_create(&th[i], NULL, span_run, &sp[i]);
    }
    for (int i = 0; i < n_threads; ++i) pthread_join(th[i], NULL);
}

typedef struct {
    int t;
    const float *x;
    uint8_t *dst;
    int64_t k;
    size_t rb;
} enc_ctx;

static void enc_span(void *p, int64_t r0, int64_t r1) {
    enc_ctx *c = (enc_ctx *)p;
    for (int64_t r = r0; r < r1; ++r) enc_row(c->t, c->x + r * c->k, c->dst + (size_t)r * c->rb, c->k);
}

int orc_quantize(int t, const float *x, void *dst, int64_t nrows, int64_t k, int n_threads) {
    const size_t rb = orc_row_size(t, k);
    if (!rb || t == ORC_BF16) return -1;
    pthread_once(&g_half_once, half_init);
    enc_ctx c = {t, x, (uint8_t *)dst, k, rb};
    par_rows(nrows, n_threads, enc_span, &c);
    return 0;
}

/* ================================================================ float activations */

/* src/matvec_q.hip:713-721 (f16_round), 805-809 (bf16_round) */
float orc_act_round(int t, int round, float x) {
    pthread_once(&g_half_once, half_init);
    if (!round || t == ORC_F32) return x;
    if (t == ORC_F16) return orc_f16_to_f32(orc_f32_to_f16(x));
    const uint32_t u = fbits(x);
    return bitsf(((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16);
}

void orc_act_round_n(int t, int round, const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_act_round(t, round, x[i]);
}

int orc_matvec_float(int t, int round, const void *W, size_t rb, int N, int K, int T, const float *x, double *ref,
                     double *mag) {
    if ((t != ORC_F32 && t != ORC_F16 && t != ORC_BF16) || rb < orc_row_size(t, K)) return -1;
    pthread_once(&g_half_once, half_init);
    float *w = (float *)malloc((size_t)K * 4), *xa = (float *)malloc((size_t)K * 4);
    if (!w || !xa) { free(w); free(xa); return -1; }
    for (int tt = 0; tt < T; ++tt) {
        for (int k = 0; k < K; ++k) xa[k] = orc_act_round(t, round, x[(size_t)tt * K + k]);
        for (int n = 0; n < N; ++n) {
            orc_to_float(t, (const uint8_t *)W + (size_t)n * rb, w, K);
            double s = 0.0, m = 0.0;
            for (int k = 0; k < K; ++k) {
                const double p = (double)w[k] * (double)xa[k];
                s += p;
                m += fabs(p);
            }
            ref[(size_t)tt * N + n] = s;
            mag[(size_t)tt * N + n] = m;
        }
    }
    free(w);
    free(xa);
    return 0;
}

/* ================================================================ activation quantizers */

/* Q8_0 activations (src/q8_device.h:54-76, src/expert_cpu.cpp:39-48): per 32 values am = max |x|
 * (fmaxf), q = rint(x * (127 / am)) ties to even, d = fp16(am / 127), and the Q8_1 sum
 * s0 = fp16((am / 127) * sum q) kept as float bits (d unrounded there). */
void orc_quantize_q8_0(const float *x, int64_t k, int8_t *q0, float *d0, int32_t *s0) {
    for (int64_t b = 0; b < k / 32; ++b) {
        const float *xb = x + 32 * b;
        float am = 0.0f;
        for (int j = 0; j < 32; ++j) am = fmaxf(am, fabsf(xb[j]));
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        int sum = 0;
        for (int j = 0; j < 32; ++j) {
            const int q = (int)rintf(xb[j] * id);
            q0[32 * b + j] = (int8_t)q;
            sum += q;
        }
        const float d = am / 127.0f;
        d0[b] = orc_f16_to_f32(orc_f32_to_f16(d));
        if (s0) {
            const float s = orc_f16_to_f32(orc_f32_to_f16(d * (float)sum));
            memcpy(&s0[b], &s, 4);
        }
    }
}

/* Q8_K activations (src/q8_device.h:78-104; tests/matvec_verify.cpp:55-66): per 256 values the signed
 * value v of largest |x| (the first on ties), iscale = -127 / v, q = min(127, rint(iscale * x)),
 * d = 1 / iscale (0 for an all-zero block), and the sum of every 16 q. */
void orc_quantize_q8_k(const float *x, int64_t k, int8_t *qK, float *dK, int32_t *bsK) {
    for (int64_t b = 0; b < k / 256; ++b) {
        const float *xb = x + 256 * b;
        float amax = 0.0f, v = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float a = fabsf(xb[j]);
            if (a > amax) {
                amax = a;
                v = xb[j];
            }
        }
        float iscale = 0.0f;
        if (amax != 0.0f) iscale = -127.0f / v;
        for (int j = 0; j < 256; ++j) {
            int q = 0;
            if (amax != 0.0f) {
                q = (int)rintf(iscale * xb[j]);
                if (q > 127) q = 127;
            }
            qK[256 * b + j] = (int8_t)q;
        }
        dK[b] = amax != 0.0f ? 1.0f / iscale : 0.0f;
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int j = 0; j < 16; ++j) s += qK[256 * b + 16 * g + j];
            bsK[16 * b + g] = s;
        }
    }
}

/* ================================================================ integer block dots */

int orc_group_size(int t) {
    switch (t) {
    case ORC_Q8_0: case ORC_FAST: case ORC_Q4_K: case ORC_Q5_K: case ORC_IQ4_XS: case ORC_MXFP4: return 32;
    case ORC_FP4: case ORC_Q6_K: case ORC_NVFP4: return 16;
    default: return 0;
    }
}

/* raw integer level of value v of a row and its weight-side dot partner: the value whose product with
 * the activation's q forms the per-group integer sum the kernels compute */
static inline int raw_level(int t, const uint8_t *row, int v) {
    switch (t) {
    case ORC_Q8_0: return (int8_t)row[34 * (v >> 5) + 2 + (v & 31)];
    case ORC_FP4: {
        const uint8_t *b = row + 18 * (v >> 5);
        const int j = v & 31;
        return k_cb[j < 16 ? (b[j] & 0xf) : (b[j - 16] >> 4)];
    }
    case ORC_FAST: {
        const uint8_t *b = row + 17 * (v >> 5);
        const int j = v & 31;
        return k_cb[j < 16 ? (b[j] & 0xf) : (b[j - 16] >> 4)];
    }
    case ORC_MXFP4: {
        const uint8_t *b = row + 17 * (v >> 5) + 1;
        const int j = v & 31;
        return k_e2m1[j < 16 ? (b[j] & 0xf) : (b[j - 16] >> 4)];
    }
    case ORC_NVFP4: {
        const uint8_t q = row[36 * (v >> 6) + 4 + 8 * ((v >> 4) & 3) + (v & 7)];
        return k_e2m1[(v & 8) ? q >> 4 : q & 0xf];
    }
    case ORC_Q4_K: return k4_level(row + 144 * (v >> 8), v & 255);
    case ORC_Q5_K: return k5_level(row + 176 * (v >> 8), v & 255);
    case ORC_IQ4_XS: return iq4xs_level(row + 136 * (v >> 8), v & 255);
    case ORC_Q6_K: return k6_level(row + 210 * (v >> 8), v & 255);
    }
    return 0;
}

int orc_block_dots(int t, const void *W, size_t rb, int N, int K, const int8_t *qx, int32_t *out) {
    const int g = orc_group_size(t);
    if (!g || K % orc_block_size(t)) return -1;
    const int ng = K / g;
    for (int n = 0; n < N; ++n) {
        const uint8_t *row = (const uint8_t *)W + (size_t)n * rb;
        for (int j = 0; j < ng; ++j) {
            int s = 0;
            for (int i = 0; i < g; ++i) s += raw_level(t, row, g * j + i) * qx[g * j + i];
            out[(size_t)n * ng + j] = s;
        }
    }
    return 0;
}

/* The exact integer a K-quant super-block contributes before its float scales (per row n and super-block u,
 * out[n * K / 256 + u]), against the Q8_K activation qK (bsK its 16-value sums):
 *   Q4_K, Q5_K  isum = sum_j sc_j dot_j over the 8 sub-blocks (raw levels)   src/matvec_q.hip:1752-1789
 *   Q6_K        isum = sum_g sc_g (dot_g - 32 bs_g) over the 16 groups       src/matvec_q.hip:1716-1750
 *   IQ4_XS      isum = sum_j (ls_j - 32) dot_j (table levels)                src/matvec_q.hip:1788-1810
 * (the reference forms these per lane and adds the lanes' floats; the sum over a super-block is the integer the
 * GEMM's epilogue scales by d dx) */
int orc_unit_isum(int t, const void *W, size_t rb, int N, int K, const int8_t *qK, const int32_t *bsK, int32_t *out) {
    if (t != ORC_Q4_K && t != ORC_Q5_K && t != ORC_Q6_K && t != ORC_IQ4_XS) return -1;
    if (K % 256) return -1;
    const int nu = K / 256, BY = t == ORC_Q4_K ? 144 : t == ORC_Q5_K ? 176 : t == ORC_Q6_K ? 210 : 136;
    for (int n = 0; n < N; ++n) {
        const uint8_t *row = (const uint8_t *)W + (size_t)n * rb;
        for (int u = 0; u < nu; ++u) {
            const uint8_t *b = row + (size_t)BY * u;
            const int8_t *xb = qK + 256 * u;
            int isum = 0;
            if (t == ORC_Q6_K) {
                const int8_t *sc = (const int8_t *)(b + 192);
                for (int g = 0; g < 16; ++g) {
                    int dot = 0;
                    for (int i = 0; i < 16; ++i) dot += k6_level(b, 16 * g + i) * xb[16 * g + i];
                    isum += sc[g] * (dot - 32 * bsK[16 * u + g]);
                }
            } else {
                for (int j = 0; j < 8; ++j) {
                    int dot = 0, sc, mn;
                    for (int i = 0; i < 32; ++i) dot += raw_level(t, row, 256 * u + 32 * j + i) * xb[32 * j + i];
                    if (t == ORC_IQ4_XS) sc = iq4xs_scale(b, j);
                    else k4_scale_min(j, b + 4, &sc, &mn);
                    isum += sc * dot;
                }
            }
            out[(size_t)n * nu + u] = isum;
        }
    }
    return 0;
}

/* ================================================================ matvec */

/* one row's result in the int8 kernels' per-block form, summed in block order:
 *   Q8_0  (e * dx) * s                               src/matvec_q.hip:1566-1573, src/expert_cpu.cpp:223-229
 *   FP4   (e0 * dx) * s0 + (e1 * dx) * s1            src/matvec_q.hip:1310-1327 (P4ROCmFP4::block)
 *   FAST  (e * dx) * (s0 + s1)                       src/matvec_q.hip:1492-1502, src/expert_cpu.cpp:50-63
 *   MXFP4 (e * dx) * (s0 + s1), e the E8M0 scale     src/matvec_q.hip:1461-1472 (PFMXFP4), 1492-1502
 *   NVFP4 per 32 values (sub-blocks 2h, 2h + 1 of a 64-block): (dx * e0) * s0 + (dx * e1) * s1
 *                                                    src/matvec_q.hip:1357-1372 (P4NVFP4::block)
 *   Q4_K  per 8 lanes of 16 bytes: (d * dx) * isum - (dmin * dx) * msum     src/matvec_q.hip:1752-1789
 *   Q5_K  the same with 5-bit levels (qh bit 2c / 2c + 1 as bit 4)           src/matvec_q.hip:1752-1789,1928-1930
 *   Q6_K  per 8 lanes of 16 bytes: (d * dx) * (isum - 32 * offs)            src/matvec_q.hip:1716-1750
 *   IQ4_XS per 8 lanes of a 32-value sub-block: (d * dx) * ((ls - 32) * dot)  src/matvec_q.hip:1788-1810 */
static float row_q8(int t, const uint8_t *row, int K, const int8_t *q, const float *d, const int32_t *bs,
                    double *mag) {
    float acc = 0.0f;
    double m = 0.0;
    if (t == ORC_Q8_0) {
        for (int ib = 0; ib < K / 32; ++ib) {
            const uint8_t *b = row + 34 * ib;
            int s = 0;
            for (int j = 0; j < 32; ++j) s += (int)(int8_t)b[2 + j] * q[32 * ib + j];
            const float term = rd16(b) * d[ib] * (float)s;
            acc += term;
            m += fabs((double)term);
        }
    } else if (t == ORC_FP4) {
        for (int ib = 0; ib < K / 32; ++ib) {
            const uint8_t *b = row + 18 * ib;
            int s0 = 0, s1 = 0;
            for (int j = 0; j < 16; ++j) {
                s0 += k_cb[b[j] & 0xf] * q[32 * ib + j];
                s1 += k_cb[b[j] >> 4] * q[32 * ib + 16 + j];
            }
            const float t0 = orc_ue4m3_half(b[16]) * d[ib] * (float)s0;
            const float t1 = orc_ue4m3_half(b[17]) * d[ib] * (float)s1;
            acc += t0 + t1;
            m += fabs((double)t0) + fabs((double)t1);
        }
    } else if (t == ORC_FAST) {
        for (int ib = 0; ib < K / 32; ++ib) {
            const uint8_t *b = row + 17 * ib;
            int s = 0;
            for (int j = 0; j < 16; ++j) s += k_cb[b[j] & 0xf] * q[32 * ib + j] + k_cb[b[j] >> 4] * q[32 * ib + 16 + j];
            const float term = orc_ue4m3_half(b[16]) * d[ib] * (float)s;
            acc += term;
            m += fabs((double)term);
        }
    } else if (t == ORC_MXFP4) {
        for (int ib = 0; ib < K / 32; ++ib) {
            const uint8_t *b = row + 17 * ib;
            int s = 0;
            for (int j = 0; j < 16; ++j)
                s += k_e2m1[b[1 + j] & 0xf] * q[32 * ib + j] + k_e2m1[b[1 + j] >> 4] * q[32 * ib + 16 + j];
            const float term = orc_e8m0_half(b[0]) * d[ib] * (float)s;
            acc += term;
            m += fabs((double)term);
        }
    } else if (t == ORC_NVFP4) {
        for (int ib = 0; ib < K / 32; ++ib) {
            const uint8_t *b = row + 36 * (ib >> 1);
            const int s0b = 2 * (ib & 1);   /* sub-blocks s0b (values 0..15) and s0b + 1 (16..31) */
            int s0 = 0, s1 = 0;
            for (int j = 0; j < 16; ++j) {
                s0 += raw_level(ORC_NVFP4, row, 32 * ib + j) * q[32 * ib + j];
                s1 += raw_level(ORC_NVFP4, row, 32 * ib + 16 + j) * q[32 * ib + 16 + j];
            }
            const float t0 = d[ib] * nv_scale(b[s0b]) * (float)s0;
            const float t1 = d[ib] * nv_scale(b[s0b + 1]) * (float)s1;
            acc += t0 + t1;
            m += fabs((double)t0) + fabs((double)t1);
        }
    } else if (t == ORC_Q4_K || t == ORC_Q5_K) {
        const int q5 = t == ORC_Q5_K, BY = q5 ? 176 : 144;
        for (int ib = 0; ib < K / 256; ++ib) {
            const uint8_t *b = row + BY * ib;
            const int8_t *xb = q + 256 * ib;
            const float dw = rd16(b), dm = rd16(b + 2), dx = d[ib];
            for (int s = 0; s < 8; ++s) {      /* lane s: 16 bytes of chunk s / 2 */
                const int c = s >> 1, l = (s & 1) * 16;
                int slo = 0, shi = 0;
                for (int i = 0; i < 16; ++i) {
                    const int vlo = q5 ? k5_level(b, 64 * c + l + i) : k4_level(b, 64 * c + l + i);
                    const int vhi = q5 ? k5_level(b, 64 * c + 32 + l + i) : k4_level(b, 64 * c + 32 + l + i);
                    slo += vlo * xb[64 * c + l + i];
                    shi += vhi * xb[64 * c + 32 + l + i];
                }
                int sc1, m1, sc2, m2, sm, mm;
                k4_scale_min(2 * c, b + 4, &sc1, &m1);
                k4_scale_min(2 * c + 1, b + 4, &sc2, &m2);
                k4_scale_min(s, b + 4, &sm, &mm);
                const int isum = sc1 * slo + sc2 * shi;
                const int msum = mm * (bs[16 * ib + 2 * s] + bs[16 * ib + 2 * s + 1]);
                const float ta = dw * dx * (float)isum, tb = dm * dx * (float)msum;
                acc += ta - tb;
                m += fabs((double)ta) + fabs((double)tb);
            }
        }
    } else if (t == ORC_IQ4_XS) {
        for (int ib = 0; ib < K / 256; ++ib) {
            const uint8_t *b = row + 136 * ib;
            const int8_t *xb = q + 256 * ib;
            const float dw = rd16(b), dx = d[ib];
            for (int s = 0; s < 8; ++s) {
                int dot = 0;
                for (int i = 0; i < 32; ++i) dot += iq4xs_level(b, 32 * s + i) * xb[32 * s + i];
                const float term = dw * dx * (float)(iq4xs_scale(b, s) * dot);
                acc += term;
                m += fabs((double)term);
            }
        }
    } else if (t == ORC_Q6_K) {
        for (int ib = 0; ib < K / 256; ++ib) {
            const uint8_t *b = row + 210 * ib;
            const int8_t *sc = (const int8_t *)(b + 192);
            const int8_t *xb = q + 256 * ib;
            const float dw = rd16(b + 208), dx = d[ib];
            for (int s = 0; s < 8; ++s) {      /* lane s: ql bytes 64 h + r .. + 15 */
                const int h = s >> 2, r = (s & 3) * 16, l = r & 31, second = r >= 32;
                const int sh = second ? 2 : 0;
                const int v_lo = 128 * h + (second ? 32 : 0) + l, v_hi = v_lo + 64;
                const int g_lo = 8 * h + l / 16 + (second ? 2 : 0), g_hi = g_lo + 4;
                int slo = 0, shi = 0;
                for (int i = 0; i < 16; ++i) {
                    const uint8_t ql = b[64 * h + r + i], qh = b[128 + 32 * h + l + i];
                    slo += ((ql & 0xf) | (((qh >> sh) & 3) << 4)) * xb[v_lo + i];
                    shi += ((ql >> 4) | (((qh >> (sh + 4)) & 3) << 4)) * xb[v_hi + i];
                }
                int isum = sc[g_lo] * slo + sc[g_hi] * shi;
                isum -= 32 * (sc[2 * s] * bs[16 * ib + 2 * s] + sc[2 * s + 1] * bs[16 * ib + 2 * s + 1]);
                const float term = dw * dx * (float)isum;
                acc += term;
                m += fabs((double)term);
            }
        }
    }
    if (mag) *mag = m;
    return acc;
}

typedef struct {
    int t;
    const uint8_t *W;
    size_t rb;
    int K;
    const int8_t *q;
    const float *d;
    const int32_t *bs;
    float *y;
    double *ref, *mag;
} mv_ctx;

static void mv_span(void *p, int64_t r0, int64_t r1) {
    mv_ctx *c = (mv_ctx *)p;
    const int kq = c->t == ORC_Q4_K || c->t == ORC_Q5_K || c->t == ORC_Q6_K || c->t == ORC_IQ4_XS;
    float *wf = c->ref ? (float *)malloc((size_t)c->K * 4) : NULL;
    for (int64_t n = r0; n < r1; ++n) {
        const uint8_t *row = c->W + (size_t)n * c->rb;
        double mg = 0.0;
        c->y[n] = row_q8(c->t, row, c->K, c->q, c->d, c->bs, &mg);
        if (c->ref) {
            orc_to_float(c->t, row, wf, c->K);
            double r = 0.0, a = 0.0;
            for (int k = 0; k < c->K; ++k) {
                const double xv = (double)c->q[k] * (double)c->d[kq ? k / 256 : k / 32];
                r += (double)wf[k] * xv;
                a += fabs((double)wf[k] * xv);
            }
            c->ref[n] = r;
            if (c->mag) c->mag[n] = a;
        } else if (c->mag) {
            c->mag[n] = mg;
        }
    }
    free(wf);
}

int orc_matvec(int t, const void *W, size_t rb, int N, int K, const int8_t *q, const float *d, const int32_t *bs,
               float *y, double *ref, double *mag, int n_threads) {
    if (!orc_group_size(t) || K % orc_block_size(t) || rb != orc_row_size(t, K)) return -1;
    mv_ctx c = {t, (const uint8_t *)W, rb, K, q, d, bs, y, ref, mag};
    par_rows(N, n_threads, mv_span, &c);
    return 0;
}

/* ================================================================ the reference CPU expert path */

/* src/expert_cpu.cpp:39-48 (its rounding of d goes through F16C: IEEE round to nearest even) */
void orc_cpu_q8_0_quantize(const float *x, int K, int8_t *q, float *d) { orc_quantize_q8_0(x, K, q, d, NULL); }

/* src/expert_cpu.cpp:50-63 (the scalar path: a block at a time, acc += (e * d) * s) */
void orc_cpu_matvec_fp4fast_q8(const void *W, size_t rb, int N, int K, const int8_t *q, const float *d, float *y) {
    for (int n = 0; n < N; ++n) y[n] = row_q8(ORC_FAST, (const uint8_t *)W + (size_t)n * rb, K, q, d, NULL, NULL);
}

/* src/expert_cpu.cpp:213-232 (scalar path) */
void orc_cpu_matvec_q8_q8(const void *W, size_t rb, int N, int K, const int8_t *q, const float *d, float *y) {
    for (int n = 0; n < N; ++n) y[n] = row_q8(ORC_Q8_0, (const uint8_t *)W + (size_t)n * rb, K, q, d, NULL, NULL);
}

/* src/expert_cpu.cpp:234-252: gate, up, SiLU(min(g, L)) * clamp(u, -L, L) with libm expf, quantize, down */
void orc_cpu_expert_ffn(const void *gate, const void *up, size_t rb_gu, const void *down, size_t rb_d, int FE, int E,
                        const int8_t *q, const float *d, float limit, float *out) {
    float *g = (float *)malloc((size_t)FE * 4), *u = (float *)malloc((size_t)FE * 4);
    float *dq = (float *)malloc((size_t)(FE / 32) * 4);
    int8_t *aq = (int8_t *)malloc((size_t)FE);
    orc_cpu_matvec_fp4fast_q8(gate, rb_gu, FE, E, q, d, g);
    orc_cpu_matvec_fp4fast_q8(up, rb_gu, FE, E, q, d, u);
    for (int i = 0; i < FE; ++i) {
        float gv = g[i], uv = u[i];
        if (limit > 0.0f) {
            gv = fminf(gv, limit);
            uv = fminf(fmaxf(uv, -limit), limit);
        }
        g[i] = gv / (1.0f + expf(-gv)) * uv;
    }
    orc_cpu_q8_0_quantize(g, FE, aq, dq);
    orc_cpu_matvec_fp4fast_q8(down, rb_d, E, FE, aq, dq, out);
    free(g); free(u); free(dq); free(aq);
}

/* ================================================================ MoE */

/* src/gpu_ops.hip:185-241 (moe_router without the shared-expert gate): softmax in float with expf,
 * n_used rounds of argmax over the remaining probabilities (the lowest index among equals), weights
 * p / max(sum p, 2^-14). The softmax sum is sequential here. */
void orc_moe_router(const float *logits, int T, int n_expert, int n_used, int32_t *ids, float *wts) {
    float *p = (float *)malloc((size_t)n_expert * 4);
    for (int t = 0; t < T; ++t) {
        const float *l = logits + (size_t)t * n_expert;
        float mx = -INFINITY;
        for (int e = 0; e < n_expert; ++e) mx = fmaxf(mx, l[e]);
        float sum = 0.0f;
        for (int e = 0; e < n_expert; ++e) {
            p[e] = expf(l[e] - mx);
            sum += p[e];
        }
        const float inv = 1.0f / sum;
        for (int e = 0; e < n_expert; ++e) p[e] *= inv;
        float sel[64];
        for (int r = 0; r < n_used; ++r) {
            int be = -1;
            float bv = -1.0f;
            for (int e = 0; e < n_expert; ++e)
                if (p[e] > bv) { bv = p[e]; be = e; }
            ids[t * n_used + r] = be;
            sel[r] = bv;
            p[be] = -INFINITY;
        }
        float ws = 0.0f;
        for (int r = 0; r < n_used; ++r) ws += sel[r];
        ws = fmaxf(ws, 6.103515625e-5f);
        for (int r = 0; r < n_used; ++r) wts[t * n_used + r] = sel[r] / ws;
    }
    free(p);
}

/* src/gpu_ops.hip:266-330 (moe_group): entries sorted by expert (stable here: by entry index), each
 * expert's run cut into tiles of up to `tile`; returns the number of tiles */
int orc_moe_group(const int32_t *ids, int T, int n_used, int n_expert, int tile, int32_t *tok_rows,
                  int32_t *pair_rows, int32_t *tile_e, int32_t *tile_start, int32_t *tile_n) {
    const int n = T * n_used;
    int *cnt = (int *)calloc((size_t)n_expert + 1, sizeof(int));
    for (int i = 0; i < n; ++i) cnt[ids[i]]++;
    int *off = (int *)calloc((size_t)n_expert + 1, sizeof(int));
    int nt = 0;
    for (int e = 0; e < n_expert; ++e) {
        off[e + 1] = off[e] + cnt[e];
        for (int k = 0; k * tile < cnt[e]; ++k) {
            tile_e[nt] = e;
            tile_start[nt] = off[e] + k * tile;
            tile_n[nt] = cnt[e] - k * tile < tile ? cnt[e] - k * tile : tile;
            ++nt;
        }
    }
    for (int i = 0; i < n; ++i) {
        const int p = off[ids[i]]++;
        tok_rows[p] = i / n_used;
        pair_rows[p] = i;
    }
    free(cnt);
    free(off);
    return nt;
}

/* src/gpu_ops.hip:245-264 (moe_combine): out = w0 d0 + w1 d1 + ... in slot order, each expert's output first
 * times es[id] when es is set (moe_combine_scaled), weights 1 when wts is NULL, then + shared * sg (+ shared
 * when sg is NULL) when shared is set. Built without contraction: every product and sum rounds on its own. */
void orc_moe_combine(const float *down, const float *wts, const float *shared, const float *sg, const int32_t *ids,
                     const float *es, float *out, int n_used, int n, int T) {
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < n; ++i) {
            const float *dd = down + (size_t)t * n_used * n + i;
            float acc;
            if (!wts) {
                acc = dd[0];
                for (int j = 1; j < n_used; ++j) acc += dd[(size_t)j * n];
            } else {
                const float *w = wts + (size_t)t * n_used;
                const int32_t *e = ids ? ids + (size_t)t * n_used : NULL;
                acc = es ? (dd[0] * es[e[0]]) * w[0] : w[0] * dd[0];
                for (int j = 1; j < n_used; ++j)
                    acc += es ? (dd[(size_t)j * n] * es[e[j]]) * w[j] : w[j] * dd[(size_t)j * n];
            }
            if (shared) acc += sg ? shared[(size_t)t * n + i] * sg[t] : shared[(size_t)t * n + i];
            out[(size_t)t * n + i] = acc;
        }
}

/* the shared expert's gate of src/gpu_ops.hip:213-229: sg = 1 / (1 + expf(-(x . w))), the dot in double */
float orc_shared_gate(const float *x, const float *w, int n) {
    double d = 0.0;
    for (int i = 0; i < n; ++i) d += (double)x[i] * (double)w[i];
    return 1.0f / (1.0f + expf(-(float)d));
}

/* src/expert_cpu.cpp:241-248 (SiLU(g) * u with libm expf; the reference's GPU swiglu, src/gpu_ops.hip:103-113,
 * is the same expression with its fast exp) */
void orc_swiglu(const float *g, const float *u, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* ================================================================ gemm_act_fp4 */

/* src/gemm_act_fp4.hip:27-157 (UE4M3 path) and tests/actfp4_verify.cpp's CPU reference: the weights
 * dequantized with fp4_common.h's decoder and rounded to fp16 (Codebook10 nibble k of line n in byte
 * n * K/2 + k/2, low nibble first; scale byte n * K/16 + k/16), products summed in double. */
void orc_gemm_act_fp4(const uint16_t *A, const uint8_t *W, const uint8_t *Ws, float *C, int M, int N, int K) {
    float *wd = (float *)malloc((size_t)K * 4);
    for (int n = 0; n < N; ++n) {
        for (int k = 0; k < K; ++k) {
            const uint8_t b = W[(size_t)n * (K / 2) + k / 2];
            const int nib = (k & 1) ? (b >> 4) : (b & 0xf);
            const float v = (float)k_cb[nib] * orc_ue4m3_fp4common(Ws[(size_t)n * (K / 16) + k / 16]);
            wd[k] = orc_f16_to_f32(orc_f32_to_f16(v));
        }
        for (int m = 0; m < M; ++m) {
            double s = 0.0;
            for (int k = 0; k < K; ++k) s += (double)orc_f16_to_f32(A[(size_t)m * K + k]) * (double)wd[k];
            C[(size_t)m * N + n] = (float)s;
        }
    }
    free(wd);
}
