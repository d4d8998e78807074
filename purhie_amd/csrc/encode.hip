// encode.hip -- the weight encoders on the GPU: fp32 rows -> GGUF blocks (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS,
// MXFP4, NVFP4, ROCmFP4, ROCmFP4_FAST) and F32 / F16 / BF16 rows, bit-identical to the reference's CPU encoders
// (src/quantize.cpp:28-64, 161-358, 362-476, 651-750, 851-974, 975-1109), which reproduce ggml's _ref quantizers
// and ROCmFPX's rocmfp4.c.
//
// One thread per block (Q8_0, ROCmFP4, FAST, MXFP4: 32 values; NVFP4: 64) or super-block (K-quants: 256). The
// searches are the reference's, step for step, in single precision: this file is compiled without
// floating-point contraction (a fused multiply-add rounds a sum of squares differently and can pick
// another scale on a tie), divisions and square roots are IEEE-rounded (hipcc's default), and nothing is
// reassociated. The ROCmFP4 scale search is the reference's outward search from the scale nearest
// max|x| / 10; every candidate it skips is one that cannot win (its clipping error alone exceeds the best).
#include <float.h>

#include "device.h"
#include "kernels.h"

#pragma clang fp contract(off)

namespace pq {

// IEEE binary32 -> binary16, round to nearest even; NaN -> 0x7E00 with its sign (src/quantize.cpp:28-43)
__device__ __host__ inline uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    __builtin_memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;
    if (ax >= 0x477ff000u) return sign | 0x7c00u;  // rounds to infinity
    if (ax >= 0x38800000u) {                        // normal half
        const uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u);
        return sign | (uint16_t)((r - 0x38000000u) >> 13);
    }
    const int e = (int)(ax >> 23);
    const int shift = 126 - e;  // subnormal half: the value is mant >> shift units of 2^-24
    if (e == 0 || shift > 24) return sign;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t r = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return sign | (uint16_t)r;
}

// binary32 -> bfloat16, round to nearest even; NaN -> quiet NaN with its sign (src/quantize.cpp:45-51)
__device__ __host__ inline uint16_t f32_to_bf16_bits(float f) {
    uint32_t x;
    __builtin_memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

__device__ inline float f16_bits_to_f32(uint16_t h) { return h2f(h); }

// ggml's nearest_int: round half to even through 1.5 * 2^23 (valid for |v| < 2^22)
__device__ inline int nearest(float v) {
    const float s = v + 12582912.f;
    int32_t i;
    __builtin_memcpy(&i, &s, 4);
    return (i & 0x007fffff) - 0x00400000;
}

__device__ inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

// ---------------------------------------------------------------- Q8_0 (src/quantize.cpp:53-64)
__device__ void enc_q8_0_block(const float *x, uint8_t *out) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(x[j]);
        amax = amax > a ? amax : a;  // (a NaN wins, as ggml's MAX)
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t h = f32_to_f16_bits(d);
    out[0] = (uint8_t)h;
    out[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 32; ++j) out[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

// ---------------------------------------------------------------- Q4_K / Q5_K (src/quantize.cpp:169-358)

// the asymmetric scale / min search of one 32-value sub-block: returns the scale, *neg_min = -min (Q4_K: nmax
// 15, rmin -1, 20 steps; Q5_K: nmax 31, rmin -0.5, 15 steps)
template <int nmax, int nstep>
__device__ float make_qkx2(const float *x, const float *w, uint8_t *L, float *neg_min, float rmin) {
    constexpr int n = 32;
    constexpr float rdelta = 0.1f;
    uint8_t Laux[32];
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
        for (int i = 0; i < n; ++i) L[i] = 0;
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = (float)nmax / (hi - lo);
    float scale = 1.0f / iscale;
    float best = 0.0f;
    for (int i = 0; i < n; ++i) {
        const int l = clampi(nearest(iscale * (x[i] - lo)), 0, nmax);
        L[i] = (uint8_t)l;
        const float diff = scale * (float)L[i] + lo - x[i];
        best += w[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < n; ++i) {
            const int l = clampi(nearest(iscale * (x[i] - lo)), 0, nmax);
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
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best = cur;
                scale = ts;
                lo = tm;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

// the super-block's levels L (0..nmax), its packed scales and mins (bytes 4..15) and d, dmin (bytes 0..3)
template <int nmax, int nstep>
__device__ void enc_kq_levels(const float *x, uint8_t *out, uint8_t *L, float rmin) {
    float w[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float s2 = 0;
        for (int l = 0; l < 32; ++l) s2 += x[32 * j + l] * x[32 * j + l];
        const float av = sqrtf(s2 / 32);
        for (int l = 0; l < 32; ++l) w[l] = av + fabsf(x[32 * j + l]);
        scales[j] = make_qkx2<nmax, nstep>(x + 32 * j, w, L + 32 * j, &mins[j], rmin);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_s = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_m = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t scl[12];
    for (int i = 0; i < 12; ++i) scl[i] = 0;
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)nearest(inv_s * scales[j]);
        uint8_t lm = (uint8_t)nearest(inv_m * mins[j]);
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
    const uint16_t hd = f32_to_f16_bits(max_scale / 63.f), hm = f32_to_f16_bits(max_min / 63.f);
    out[0] = (uint8_t)hd;
    out[1] = (uint8_t)(hd >> 8);
    out[2] = (uint8_t)hm;
    out[3] = (uint8_t)(hm >> 8);
    for (int i = 0; i < 12; ++i) out[4 + i] = scl[i];
    const float fd = f16_bits_to_f32(hd), fm = f16_bits_to_f32(hm);
    for (int j = 0; j < 8; ++j) {
        int sc, mn;
        if (j < 4) {
            sc = scl[j] & 63;
            mn = scl[j + 4] & 63;
        } else {
            sc = (scl[j + 4] & 0xf) | ((scl[j - 4] >> 6) << 4);
            mn = (scl[j + 4] >> 4) | ((scl[j] >> 6) << 4);
        }
        const float d = fd * (float)sc;
        if (d == 0.0f) continue;
        const float dm = fm * (float)mn;
        for (int i = 0; i < 32; ++i) L[32 * j + i] = (uint8_t)clampi(nearest((x[32 * j + i] + dm) / d), 0, nmax);
    }
}

__device__ void enc_q4_k_block(const float *x, uint8_t *out) {
    uint8_t L[256];
    enc_kq_levels<15, 20>(x, out, L, -1.0f);
    uint8_t *q = out + 16;
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) q[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
}

// Q5_K: the low 4 bits as Q4_K's nibbles (bytes 48..175), bit 4 of value 64 c + l in qh byte l bit 2 c, of value
// 64 c + 32 + l in bit 2 c + 1 (bytes 16..47)
__device__ void enc_q5_k_block(const float *x, uint8_t *out) {
    uint8_t L[256];
    enc_kq_levels<31, 15>(x, out, L, -0.5f);
    uint8_t *qh = out + 16, *ql = out + 48;
    for (int l = 0; l < 32; ++l) {
        uint32_t h = 0;
        for (int c = 0; c < 4; ++c) h |= (uint32_t)((L[64 * c + l] >> 4) << (2 * c)) | ((L[64 * c + 32 + l] >> 4) << (2 * c + 1));
        qh[l] = (uint8_t)h;
    }
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) ql[32 * c + l] = (uint8_t)((L[64 * c + l] & 0xf) | ((L[64 * c + 32 + l] & 0xf) << 4));
}

// ---------------------------------------------------------------- Q6_K (src/quantize.cpp:362-476)

// the symmetric search of one 16-value group (rmse_type 1, no importance): L receives levels + 32
__device__ float make_qx(const float *x, int8_t *L) {
    constexpr int n = 16, nmax = 32;
    float mx = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) {
            amax = a;
            mx = x[i];
        }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = (float)(-nmax) / mx;
    float slx = 0, sl2 = 0;
    for (int i = 0; i < n; ++i) {
        const int l = clampi(nearest(iscale * x[i]), -nmax, nmax - 1);
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
            const int l = clampi(nearest(iscale * x[i]), -nmax, nmax - 1);
            const float w = x[i] * x[i];
            slx += w * x[i] * (float)l;
            sl2 += w * (float)l * (float)l;
        }
        if (sl2 > 0 && slx * slx > best * sl2) {
            for (int i = 0; i < n; ++i) L[i] = (int8_t)(nmax + clampi(nearest(iscale * x[i]), -nmax, nmax - 1));
            scale = slx / sl2;
            best = scale * slx;
        }
    }
    return scale;
}

__device__ void enc_q6_k_block(const float *x, uint8_t *out) {
    int8_t L[256];
    float scales[16];
    float max_scale = 0, max_abs = 0;
    for (int g = 0; g < 16; ++g) {
        const float s = make_qx(x + 16 * g, L + 16 * g);
        scales[g] = s;
        if (fabsf(s) > max_abs) {
            max_abs = fabsf(s);
            max_scale = s;
        }
    }
    for (int i = 0; i < 210; ++i) out[i] = 0;
    if (max_abs < 1e-15f) return;
    const float iscale = -128.f / max_scale;
    const uint16_t hd = f32_to_f16_bits(1.0f / iscale);
    out[208] = (uint8_t)hd;
    out[209] = (uint8_t)(hd >> 8);
    int8_t *sc = (int8_t *)(out + 192);
    for (int g = 0; g < 16; ++g) {
        const int v = nearest(iscale * scales[g]);
        sc[g] = (int8_t)(v < 127 ? v : 127);
    }
    const float fd = f16_bits_to_f32(hd);
    for (int g = 0; g < 16; ++g) {
        const float d = fd * (float)sc[g];
        if (d == 0.0f) continue;
        for (int i = 0; i < 16; ++i) L[16 * g + i] = (int8_t)(clampi(nearest(x[16 * g + i] / d), -32, 31) + 32);
    }
    uint8_t *ql = out, *qh = out + 128;
    for (int h = 0; h < 2; ++h) {
        const int8_t *Lh = L + 128 * h;
        for (int l = 0; l < 32; ++l) {
            ql[l] = (uint8_t)((Lh[l] & 0xf) | ((Lh[l + 64] & 0xf) << 4));
            ql[l + 32] = (uint8_t)((Lh[l + 32] & 0xf) | ((Lh[l + 96] & 0xf) << 4));
            qh[l] = (uint8_t)((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) | ((Lh[l + 96] >> 4) << 6));
        }
        ql += 64;
        qh += 32;
    }
}

// ---------------------------------------------------------------- ROCmFP4 / FAST (src/quantize.cpp:975-1109)

// the half-scale value of a UE4M3 byte 0..126 (0x7F and above: 0)
__device__ inline float scale_half(int e) {
    if (e > 0x7e) return 0.0f;
    return e < 8 ? ldexpf((float)e, -10) : ldexpf((float)(8 + (e & 7)), (e >> 3) - 11);
}

// Codebook10 magnitude index of |x inv|: at each midpoint the lower magnitude
__device__ inline int mag_index(float a) {
    if (a <= 0.5f) return 0;
    if (a <= 1.5f) return 1;
    if (a <= 2.5f) return 2;
    if (a <= 3.5f) return 3;
    if (a <= 5.0f) return 4;
    if (a <= 7.0f) return 5;
    if (a <= 9.0f) return 6;
    return 7;
}

__device__ inline float mag_value(int m) {
    return m < 5 ? (float)m : m == 5 ? 6.0f : m == 6 ? 8.0f : 10.0f;
}

__device__ inline uint8_t fp4_code(float x, float inv) {
    if (!isfinite(x)) return 0;
    const int m = mag_index(fabsf(x * inv));
    if (m == 0) return 0;
    return (uint8_t)(x < 0.0f ? (m | 8) : m);
}

// squared error of n values at scale byte e, given up (a value above cap) once above cap
__device__ float fp4_err(const float *x, int n, int e, float cap) {
    const float s = scale_half(e);
    const float inv = 1.0f / s;
    float err = 0.0f;
    for (int i = 0; i < n; ++i) {
        float y = 0.0f;
        if (isfinite(x[i])) {
            const float m = mag_value(mag_index(fabsf(x[i] * inv)));
            y = (x[i] < 0.0f ? -m : m) * s;
        }
        const float d = x[i] - y;
        err += d * d;
        if (err > cap) return err;
    }
    return err;
}

// the byte in 1..126 whose scale is nearest target (the lower one on a tie)
__device__ int nearest_scale(float target) {
    if (!(target > 0.0f) || !isfinite(target)) return 1;
    int lo = 1, hi = 126;
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (scale_half(mid) < target) lo = mid + 1;
        else hi = mid;
    }
    if (lo == 1) return 1;
    const float up = scale_half(lo), dn = scale_half(lo - 1);
    return (target - dn <= up - target) ? lo - 1 : lo;
}

__device__ uint8_t choose_scale(const float *x, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    if (!(amax > 0.0f) || !isfinite(amax)) return 0;
    const int start = nearest_scale(amax / 10.0f);
    int best_e = 0;
    float best = FLT_MAX;
    bool down_done = false;
    for (int delta = 0; delta <= 125; ++delta) {
        const int e0 = start - delta;
        if (!down_done && e0 >= 1 && e0 <= 126) {
            const float clip = amax - 10.0f * scale_half(e0);
            if (clip > 0.0f && clip * clip > best) {
                down_done = true;
            } else {
                const float err = fp4_err(x, n, e0, best);
                if (err < best || (err == best && e0 < best_e)) {
                    best = err;
                    best_e = e0;
                }
            }
        }
        const int e1 = start + delta;
        if (delta != 0 && e1 >= 1 && e1 <= 126) {
            const float err = fp4_err(x, n, e1, best);
            if (err < best || (err == best && e1 < best_e)) {
                best = err;
                best_e = e1;
            }
        }
        if ((down_done || e0 <= 1) && e1 >= 126) break;
    }
    return (uint8_t)best_e;
}

__device__ inline float inv_of(uint8_t e) {
    const float s = scale_half(e);
    return s > 0.0f ? 1.0f / s : 0.0f;
}

__device__ void enc_fp4_block(const float *x, uint8_t *out) {
    const uint8_t e0 = choose_scale(x, 16), e1 = choose_scale(x + 16, 16);
    const float i0 = inv_of(e0), i1 = inv_of(e1);
    for (int j = 0; j < 16; ++j) out[j] = (uint8_t)(fp4_code(x[j], i0) | (fp4_code(x[j + 16], i1) << 4));
    out[16] = e0;
    out[17] = e1;
}

__device__ void enc_fast_block(const float *x, uint8_t *out) {
    const uint8_t e = choose_scale(x, 32);
    const float inv = inv_of(e);
    for (int j = 0; j < 16; ++j) out[j] = (uint8_t)(fp4_code(x[j], inv) | (fp4_code(x[j + 16], inv) << 4));
    out[16] = e;
}

// ---------------------------------------------------------------- MXFP4 / NVFP4 (src/quantize.cpp:651-750)

__constant__ float k_e2m1f[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};  // E2M1 at half scale

// ggml's best_index_mxfp4: the first index whose level times e is nearest x (a NaN x: every error is NaN, 0)
__device__ inline uint8_t e2m1_index(float x, float e) {
    int best = 0;
    float best_err = fabsf(k_e2m1f[0] * e - x);
    for (int i = 1; i < 16; ++i) {
        const float err = fabsf(k_e2m1f[i] * e - x);
        if (err < best_err) {
            best = i;
            best_err = err;
        }
    }
    return (uint8_t)best;
}

// floor(log2f(a)) as the host's libm gives it. It differs from the exponent of a only where a lies a few units
// below a power of two and log2f rounds up to the integer; there log2f equals the double log2 rounded to float,
// which is what this returns (the two floors agree for every positive finite float, checked on the host).
__device__ inline float floor_log2f(float a) { return floorf((float)log2((double)a)); }

// float -> uint8_t as an x86-64 build converts it: truncation to int32 (out of range or NaN: INT_MIN), low byte
__device__ inline uint8_t x86_u8(float v) {
    const int i = (v >= -2147483648.0f && v < 2147483648.0f) ? (int)v : (int)0x80000000u;
    return (uint8_t)i;
}

// MXFP4: e = floor(log2(amax)) - 2 + 127, d = 2^(e - 128), each value's nearest level
__device__ void enc_mxfp4_block(const float *x, uint8_t *out) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j)
        if (amax < fabsf(x[j])) amax = fabsf(x[j]);
    const uint8_t e = amax > 0.0f ? x86_u8(floor_log2f(amax) - 2 + 127) : 0;
    const float d = e8m0_half(e);
    out[0] = e;
    for (int j = 0; j < 16; ++j) out[1 + j] = (uint8_t)(e2m1_index(x[j], d) | (e2m1_index(x[16 + j], d) << 4));
}

// ggml_fp32_to_ue4m3: nearest on the fp32 bits (the bit below the kept 3 decides), clamped to 448 and the code
// 0x7E, subnormal codes m = (int)(x * 512 + 0.5)
__device__ inline uint8_t f32_to_ue4m3(float x) {
    if (!(x > 0.0f)) return 0;
    if (x > 448.0f) x = 448.0f;
    const uint32_t bits = __float_as_uint(x);
    int e = (int)((bits >> 23) & 0xffu) - 120;
    if (e <= 0) {
        int m = (int)(x * 512.0f + 0.5f);
        if (m > 7) m = 7;
        return m < 1 ? 0 : (uint8_t)m;
    }
    if (e >= 15) return 0x7e;
    int m = (int)((bits >> 20) & 7u) + (int)((bits >> 19) & 1u);
    if (m > 7) {
        m = 0;
        if (++e >= 15) return 0x7e;
    }
    return (uint8_t)((e << 3) | m);
}

// NVFP4: per 16 values the UE4M3 code of amax / 6 and each value's nearest level at its half-scale value
__device__ void enc_nvfp4_block(const float *x, uint8_t *out) {
    for (int s = 0; s < 4; ++s) {
        const float *xb = x + 16 * s;
        float amax = 0.0f;
        for (int j = 0; j < 16; ++j)
            if (amax < fabsf(xb[j])) amax = fabsf(xb[j]);
        const uint8_t ue = f32_to_ue4m3(amax / 6.0f);
        const float d = ue4m3_half(ue);
        out[s] = ue;
        for (int j = 0; j < 8; ++j)
            out[4 + 8 * s + j] = (uint8_t)(e2m1_index(xb[j], d) | (e2m1_index(xb[8 + j], d) << 4));
    }
}

// ---------------------------------------------------------------- IQ4_XS (src/quantize.cpp:851-974)

__constant__ int8_t k_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// the nearest codebook value's index, the lower one on a tie (ggml's best_index_int8 over the sorted table)
__device__ int iq4_index(float x) {
    if (x <= (float)k_iq4nl[0]) return 0;
    if (x >= (float)k_iq4nl[15]) return 15;
    int lo = 0, hi = 15;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (x < (float)k_iq4nl[mid]) hi = mid;
        else lo = mid;
    }
    return x - (float)k_iq4nl[hi - 1] < (float)k_iq4nl[hi] - x ? hi - 1 : hi;
}

// ggml's quantize_row_iq4_nl_impl for one 256-value super-block, no importance weights, 7 retries: per 32-value
// sub-block, weights x^2, a first scale from the signed largest value, its least-squares refinement, then 15
// candidate inverse scales (itry - 127) / max keeping the largest sumqx^2 / sumq2; the sub-block scales quantized
// to 6 bits against d = -max_scale / 32 (fp32; its fp16 rounding is only stored) and every value re-indexed
__device__ void enc_iq4_xs_block(const float *x, uint8_t *out) {
    uint8_t L[256];
    float scales[8];
    float max_scale = 0, amax_scale = 0;
    for (int i = 0; i < 256; ++i) L[i] = 0;
    for (int ib = 0; ib < 8; ++ib) {
        const float *xb = x + 32 * ib;
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
            const float q = (float)k_iq4nl[l], w = xb[j] * xb[j];
            sumqx += w * q * xb[j];
            sumq2 += w * q * q;
        }
        d = sumq2 > 0 ? sumqx / sumq2 : 0.f;
        float best = d * sumqx;
        for (int itry = -7; itry <= 7; ++itry) {
            id = ((float)itry + (float)k_iq4nl[0]) / mx;
            sumqx = sumq2 = 0;
            for (int j = 0; j < 32; ++j) {
                const float q = (float)k_iq4nl[iq4_index(id * xb[j])], w = xb[j] * xb[j];
                sumqx += w * q * xb[j];
                sumq2 += w * q * q;
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
    const uint16_t dh = f32_to_f16_bits(d);
    const float id = d != 0.0f ? 1 / d : 0.f;
    uint32_t sh = 0, sl = 0;
    for (int ib = 0; ib < 8; ++ib) {
        const int l = clampi(nearest(id * scales[ib]), -32, 31);
        const float dl = d * (float)l;
        const float idl = dl != 0.0f ? 1 / dl : 0.f;
        for (int j = 0; j < 32; ++j) L[32 * ib + j] = (uint8_t)iq4_index(idl * x[32 * ib + j]);
        const uint32_t u = (uint32_t)(l + 32);
        sl |= (u & 0xfu) << (4 * ib);
        sh |= (u >> 4) << (2 * ib);
    }
    out[0] = (uint8_t)dh;
    out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)sh;
    out[3] = (uint8_t)(sh >> 8);
    for (int i = 0; i < 4; ++i) out[4 + i] = (uint8_t)(sl >> (8 * i));
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 16; ++j) out[8 + 16 * i + j] = (uint8_t)(L[32 * i + j] | (L[32 * i + 16 + j] << 4));
}

// ---------------------------------------------------------------- kernels

// one thread per block of `vals` values: block i of row r at x + r * ncols + i * vals
template <int TYPE>
__global__ void __launch_bounds__(256) k_encode(const float *__restrict__ x, uint8_t *__restrict__ y, long long nrows,
                                                long long ncols, long long row_bytes) {
    constexpr int VALS = (TYPE == TY_Q4_K || TYPE == TY_Q5_K || TYPE == TY_Q6_K || TYPE == TY_IQ4_XS) ? 256
                         : TYPE == TY_NVFP4                                                          ? 64
                                                                                                      : 32;
    constexpr int BYTES = TYPE == TY_Q8_0   ? 34
                          : TYPE == TY_Q4_K ? 144
                          : TYPE == TY_Q5_K ? 176
                          : TYPE == TY_Q6_K ? 210
                          : TYPE == TY_IQ4_XS ? 136
                          : TYPE == TY_NVFP4 ? 36
                          : TYPE == TY_FP4  ? 18
                                            : 17;
    const long long per_row = ncols / VALS;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * per_row) return;
    const long long r = i / per_row, b = i - r * per_row;
    const float *src = x + r * ncols + b * VALS;
    uint8_t *dst = y + r * row_bytes + b * BYTES;
    if (TYPE == TY_Q8_0) enc_q8_0_block(src, dst);
    else if (TYPE == TY_Q4_K) enc_q4_k_block(src, dst);
    else if (TYPE == TY_Q5_K) enc_q5_k_block(src, dst);
    else if (TYPE == TY_IQ4_XS) enc_iq4_xs_block(src, dst);
    else if (TYPE == TY_Q6_K) enc_q6_k_block(src, dst);
    else if (TYPE == TY_FP4) enc_fp4_block(src, dst);
    else if (TYPE == TY_MXFP4) enc_mxfp4_block(src, dst);
    else if (TYPE == TY_NVFP4) enc_nvfp4_block(src, dst);
    else enc_fast_block(src, dst);
}

// F16 (kind 1) / BF16 (kind 2) / F32 (kind 0) rows, one thread per value
__global__ void k_encode_float(const float *__restrict__ x, uint8_t *__restrict__ y, long long n, int kind) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (kind == 0) ((float *)y)[i] = x[i];
    else ((uint16_t *)y)[i] = kind == 1 ? f32_to_f16_bits(x[i]) : f32_to_bf16_bits(x[i]);
}

// values per block of an encodable type (0: not one of them); F32 / F16 / BF16: 1
int encode_block_values(int type) {
    switch (type) {
    case 0: case 1: case 30: return 1;
    case TY_Q8_0: case TY_FP4: case TY_FAST: case TY_MXFP4: return 32;
    case TY_NVFP4: return 64;
    case TY_Q4_K: case TY_Q5_K: case TY_Q6_K: case TY_IQ4_XS: return 256;
    }
    return 0;
}

hipError_t launch_encode(int type, const float *x, uint8_t *y, long long nrows, long long ncols, long long row_bytes,
                         hipStream_t stream) {
    const int vals = encode_block_values(type);
    if (!vals || ncols % vals) return hipErrorInvalidValue;
    const long long n = nrows * (ncols / vals);
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (type) {
    case 0: hipLaunchKernelGGL(k_encode_float, grid, dim3(256), 0, stream, x, y, n, 0); break;
    case 1: hipLaunchKernelGGL(k_encode_float, grid, dim3(256), 0, stream, x, y, n, 1); break;
    case 30: hipLaunchKernelGGL(k_encode_float, grid, dim3(256), 0, stream, x, y, n, 2); break;
    case TY_Q8_0: hipLaunchKernelGGL(k_encode<TY_Q8_0>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes); break;
    case TY_Q4_K: hipLaunchKernelGGL(k_encode<TY_Q4_K>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes); break;
    case TY_Q5_K: hipLaunchKernelGGL(k_encode<TY_Q5_K>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes); break;
    case TY_IQ4_XS:
        hipLaunchKernelGGL(k_encode<TY_IQ4_XS>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes);
        break;
    case TY_Q6_K: hipLaunchKernelGGL(k_encode<TY_Q6_K>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes); break;
    case TY_FP4: hipLaunchKernelGGL(k_encode<TY_FP4>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes); break;
    case TY_FAST: hipLaunchKernelGGL(k_encode<TY_FAST>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes); break;
    case TY_MXFP4:
        hipLaunchKernelGGL(k_encode<TY_MXFP4>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes);
        break;
    case TY_NVFP4:
        hipLaunchKernelGGL(k_encode<TY_NVFP4>, grid, dim3(256), 0, stream, x, y, nrows, ncols, row_bytes);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

uint16_t host_f32_to_f16(float f) { return f32_to_f16_bits(f); }
uint16_t host_f32_to_bf16(float f) { return f32_to_bf16_bits(f); }

// ---------------------------------------------------------------- FP8 (OCP e4m3fn) rows with block scales
// e4m3fn: sign, 4 exponent bits (bias 7), 3 mantissa bits, no infinities, S.1111.111 NaN: exponent field 0 is
// m 2^-9, else (8 + m) 2^(e - 10) = 1.m 2^(e - 7) (the reference's qz_fp8_e4m3_to_fp32, src/quantize.cpp:1224-1233)
__device__ __host__ inline float fp8_e4m3fn(uint32_t v) {
    const uint32_t e = (v >> 3) & 15u, m = v & 7u;
    uint32_t bits;
    if ((v & 0x7fu) == 0x7fu) {
        bits = 0x7fc00000u;
    } else if (e == 0) {
        const float f = (float)m * 0x1p-9f;  // exact
        __builtin_memcpy(&bits, &f, 4);
    } else {
        bits = ((e + 120u) << 23) | (m << 20);
    }
    bits |= (v & 0x80u) << 24;
    float f;
    __builtin_memcpy(&f, &bits, 4);
    return f;
}

float host_fp8_e4m3fn(uint8_t v) { return fp8_e4m3fn(v); }

// rows r0 .. r0 + nrows - 1 of the source (this chunk: src and out start at row r0): out[r][j] = fp8(src[r][j]) *
// scale[(r0 + r) / block_rows][j / block_cols], one rounding (src/quantize.cpp:1241-1258). A NaN code stays its
// own NaN (sign included), as the host's multiply returns a NaN operand unchanged.
__global__ void __launch_bounds__(256) k_fp8_blocks(const uint8_t *__restrict__ src, const float *__restrict__ scale,
                                                    float *__restrict__ out, long long nrows, long long ncols,
                                                    long long r0, int block_rows, int block_cols,
                                                    long long scale_cols) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= nrows * ncols) return;
    const long long r = i / ncols, j = i - r * ncols;
    const uint32_t v = src[i];
    const float f = fp8_e4m3fn(v);
    out[i] = (v & 0x7fu) == 0x7fu ? f : f * scale[((r0 + r) / block_rows) * scale_cols + j / block_cols];
}

hipError_t launch_fp8_blocks(const uint8_t *src, const float *scale, float *out, long long nrows, long long ncols,
                             long long r0, int block_rows, int block_cols, long long scale_cols, hipStream_t stream) {
    const long long n = nrows * ncols;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fp8_blocks, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, src, scale, out, nrows,
                       ncols, r0, block_rows, block_cols, scale_cols);
    return hipGetLastError();
}

}  // namespace pq
