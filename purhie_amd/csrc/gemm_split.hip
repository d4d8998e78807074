// Prefill GEMM for the FP4 types with UE4M3 scales (ROCmFP4, ROCmFP4_FAST, NVFP4): y[t][n] = sum_k W[n][k] X[t][k]
// for a Q8_0 activation X = q0 d0, read in place (no pre-pass, no workspace).
//
// The reference's WMMA kernels (src/matvec_q.hip:2566-2973, src/qmatvec.cpp:444-520) take the block dot per 32
// values and scale it by d_w d_x. Here the weight value CB * scale is an fp16 number (a codebook level of at most 12
// times a UE4M3 half-scale in [2^-10, 240]: at most 8 significant bits, inside the fp16 range), so the weights go
// to the matrix core as they are, and the per-block activation scale is folded into the token operand instead:
// X 2^s = hi + lo with hi = fp16(q ds), lo = fp16(q ds - hi), ds = fp16(d0 2^s), and s a per-token power of two that
// puts the token's largest |X| just under 2^14. hi + lo carries X to 2^-22 relative (the lo rounding), the products
// with the fp16 weights are exact in fp32, and the f16 MFMAs accumulate straight through K with no per-block
// epilogue: y = (sum_k W[n][k] (hi + lo)[t][k]) 2^-s. A per-block fp32 epilogue would cost one VALU fma per output
// per block, as many VALU cycles as the block's MFMAs take; the second plane costs MFMA cycles instead, with the
// VALU left for staging.
//
// Workgroup: 512 threads (8 waves) over 256 weight rows x TT tokens, K in stages of 64 (two 32-value blocks),
// double-buffered in LDS with one barrier per stage; every global load is issued two stages before its LDS store.
// Staging: thread t decodes block (t & 1) of weight row t / 2 through a byte -> (level, level) table, times the
// block's scales, into fp16; the token rows go to LDS as fp16 integers in the weight's K order (per 32-block,
// position 2j <- value j, 2j + 1 <- value j + 16: one weight byte holds values j and j + 16), with each (token,
// block) scale ds. Each wave makes the hi and lo fragments of its token tiles from them and runs the MFMAs.
#include "device.h"
#include "kernels.h"

namespace pq {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int SP_THREADS = 512;
constexpr int SP_ROWS = 256;         // weight rows per workgroup
constexpr int SP_K = 64;             // K per stage
constexpr int SP_ROW = SP_K + 8;     // halves per LDS row (16 bytes of padding: conflict-free 16-byte fragment reads)
constexpr int SP_T = 256;            // tokens per workgroup, dense
constexpr int SP_T_SMALL = 64;       // MoE expert tiles (a few dozen entries on average) and prompts of <= 64 tokens
constexpr int SP_GROUP = 4;          // token tiles advancing together over the row tiles (XCD order)

// wave layout: WC waves along the tokens, 8 / WC along the rows; each wave RT x CT tiles of 16 x 16
template <int TT>
struct SpGeo {
    static constexpr int WC = TT >= 256 ? 4 : 2;
    static constexpr int WR = 8 / WC;
    static constexpr int RT = SP_ROWS / (16 * WR);
    static constexpr int CT = TT / (16 * WC);
    static constexpr int TPR = SP_THREADS / TT;  // staging threads per token row
    static constexpr int VJ = 32 / TPR;          // (j, j + 16) value pairs a staging thread converts per stage
    static_assert(RT * 16 * WR == SP_ROWS && CT * 16 * WC == TT && VJ >= 4, "tile geometry");
};

// one 32-value FP4 block: 16 code bytes (4 words, byte i: codes of values i low and i + 16 high) and the two
// half-block scales -> 16 half2 (value i, value i + 16) in LDS through the byte -> (level, level) table; the scales
// are fp16 values (UE4M3 at half scale lies in [2^-10, 240]) and a level times one is exact
__device__ __forceinline__ void fp4_block_to_lds(const uint32_t qs[4], float e0, float e1, const uint32_t *lut,
                                                 _Float16 *dst) {
    h2 sc;
    sc.x = (_Float16)e0;
    sc.y = (_Float16)e1;
    uint32_t o[16];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const h2 c = __builtin_bit_cast(h2, lut[(qs[k] >> (8 * j)) & 0xffu]);
            o[4 * k + j] = __builtin_bit_cast(uint32_t, c * sc);  // v_pk_mul_f16: exact products
        }
    uint4 *d4 = (uint4 *)dst;
#pragma unroll
    for (int m = 0; m < 4; ++m) d4[m] = make_uint4(o[4 * m], o[4 * m + 1], o[4 * m + 2], o[4 * m + 3]);
}

// one thread's weight block per stage: raw global words, then the decode into 32 fp16 values in LDS
template <int TYPE>
struct SpW {
    static constexpr int TOP = 10;
    static constexpr int BB = TYPE == TY_FP4 ? 18 : 17;  // block bytes: 16 of codes, then 2 (1) UE4M3 scale bytes
    struct Raw {
        uint32_t w[5];
        uint32_t off;
    };
    // block 2 s + h of the row: five words from the 4-aligned address at or below it (they end at most 3 bytes
    // past the block, inside the 4-aligned word that holds its last byte)
    __device__ static void load(const uint8_t *row, int s, int h, Raw &r) {
        const uint8_t *b = row + (long long)(2 * s + h) * BB;
        r.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *al = b - r.off;
#pragma unroll
        for (int k = 0; k < 5; ++k) r.w[k] = ld32(al + 4 * k);
    }
    __device__ static void decode(const Raw &r, const uint32_t *lut, _Float16 *dst) {
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = align_bytes(r.w[k + 1], r.w[k], r.off);
        const uint32_t sc = r.w[4] >> (8 * r.off);  // the scale bytes at block offset 16 (and 17)
        const float e0 = ue4m3_half(sc);
        const float e1 = TYPE == TY_FP4 ? ue4m3_half(sc >> 8) : e0;
        fp4_block_to_lds(v, e0, e1, lut, dst);
    }
};

// NVFP4: 36-byte blocks of 64 values (4 UE4M3 scale bytes, then four 16-value sub-blocks of 8 bytes, byte i: values
// i low, 8 + i high). Stage s is block s; half h (sub-blocks 2h, 2h + 1) is regrouped into the ROCmFP4 byte order of
// a 32-value block (byte i: value i low, value 16 + i high) with the two sub-block scales as its half-block scales.
template <>
struct SpW<TY_NVFP4> {
    static constexpr int TOP = 12;
    struct Raw {
        uint32_t sc, v[4];
    };
    __device__ static void load(const uint8_t *row, int s, int h, Raw &r) {
        const uint8_t *b = row + (long long)s * 36;
        r.sc = ld32(b) >> (16 * h);
#pragma unroll
        for (int k = 0; k < 4; ++k) r.v[k] = ld32(b + 4 + 16 * h + 4 * k);
    }
    __device__ static void decode(const Raw &r, const uint32_t *lut, _Float16 *dst) {
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t lo = r.v[k], hi = r.v[2 + k];
            q[k] = (lo & 0x0f0f0f0fu) | ((hi & 0x0f0f0f0fu) << 4);
            q[2 + k] = ((lo >> 4) & 0x0f0f0f0fu) | (hi & 0xf0f0f0f0u);
        }
        fp4_block_to_lds(q, nv_scale(r.sc), nv_scale(r.sc >> 8), lut, dst);
    }
};

// four (value j, value j + 16) pairs of int8 from words a (values j .. j + 3) and b (values j + 16 .. j + 19) as four
// fp16 pairs: the byte b ^ 0x80 under 0x64 is the fp16 1024 + 128 + b, minus 1152
__device__ __forceinline__ void pairs_to_h2(uint32_t a, uint32_t b, uint32_t *o) {
    h2 bias;
    bias.x = (_Float16)1152.0f;
    bias.y = (_Float16)1152.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t w = __builtin_amdgcn_perm(b, a, 0x0c040c00u + 0x00010001u * (uint32_t)m) ^ 0x64806480u;
        o[m] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w) - bias);
    }
}

template <int N>
struct Words {
    uint32_t w[N];
};

template <int N>
__device__ __forceinline__ Words<N> load_words(const int8_t *p) {
    Words<N> r;
    if constexpr (N == 4) {
        const uint4 v = *(const uint4 *)p;
        r.w[0] = v.x;
        r.w[1] = v.y;
        r.w[2] = v.z;
        r.w[3] = v.w;
    } else if constexpr (N == 2) {
        const uint2 v = *(const uint2 *)p;
        r.w[0] = v.x;
        r.w[1] = v.y;
    } else {
        r.w[0] = *(const uint32_t *)p;
    }
    return r;
}

template <int V>
using IC = std::integral_constant<int, V>;

template <int B, class T>
__device__ __forceinline__ T &pick2(T &a, T &b) {
    if constexpr (B) return b;
    else return a;
}

template <int TYPE, int TT, bool MOE>
__global__ void __launch_bounds__(SP_THREADS, 1) k_gemm_split(GemmArgs a) {
    using S = SpW<TYPE>;
    using G = SpGeo<TT>;
    constexpr int TPR = G::TPR, VJ = G::VJ, NW = VJ / 4;
    __shared__ __attribute__((aligned(16))) _Float16 sW0[SP_ROWS * SP_ROW], sW1[SP_ROWS * SP_ROW];
    __shared__ __attribute__((aligned(16))) _Float16 sX0[TT * SP_ROW], sX1[TT * SP_ROW];
    __shared__ uint16_t sD0[TT * 2], sD1[TT * 2];  // ds of (token, block of the stage), fp16 bits
    __shared__ float sT[TT];                       // 2^-s per token
    __shared__ uint32_t lut[256];

    int n0, e = 0;
    const int32_t *rows = nullptr, *orow = nullptr;
    int tbase = 0, tn = 0;
    if constexpr (MOE) {  // grid (row tiles, tiles)
        const int k = blockIdx.y;
        if (k >= *a.n_tiles) return;
        e = a.tile_e[k];
        const int st = a.tile_start[k];
        rows = a.in_rows + st;
        orow = a.out_rows + st;
        tn = a.tile_n[k];
        n0 = blockIdx.x * SP_ROWS;
    } else {  // grid (token tiles, row tiles), renumbered XCD by XCD
        int tt, rt;
        xcd_tile(tt, rt, SP_GROUP);
        tbase = tt * TT;
        n0 = rt * SP_ROWS;
    }
    // token row of tile position j: real rows for j < n (dense: < T), else a repeat of a valid row whose outputs are
    // not stored
    auto trow = [&](int j) -> long long {
        if constexpr (MOE) return rows[j < tn ? j : 0];
        const int t = tbase + j;
        return t < a.T ? t : a.T - 1;
    };

    const int K = a.K, nst = K / SP_K, nb = K / 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 256) {
        const int lo = fp4_level<S::TOP>(tid & 15), hi = fp4_level<S::TOP>(tid >> 4);
        h2 v;
        v.x = (_Float16)(float)lo;
        v.y = (_Float16)(float)hi;
        lut[tid] = __builtin_bit_cast(uint32_t, v);
    }

    // staging roles. Weights: block wh = tid & 1 of row n0 + tid / 2 (rows past the end repeat the last; their
    // outputs are not stored). Tokens: row xr = tid / TPR, pairs j0 .. j0 + VJ - 1 of block xb of each stage.
    const int wr = n0 + (tid >> 1), wh = tid & 1;
    const uint8_t *wrow = a.W + ((long long)e * a.N + (wr < a.N ? wr : a.N - 1)) * a.row_bytes;
    const int xr = tid / TPR, xp = tid % TPR, xb = xp / (TPR / 2), j0 = (xp % (TPR / 2)) * VJ;
    const long long xrow = trow(xr);
    const int8_t *xsrc = a.xq + xrow * K + 32 * xb + j0;
    const float *dsrc = a.dx + xrow * nb + xb;

    struct Pre {
        typename S::Raw raw;
        Words<NW> qa, qb;
        float d;
    };
    Pre P0, P1;
    auto issue = [&](Pre &p, int s) {
        S::load(wrow, s, wh, p.raw);
        p.qa = load_words<NW>(xsrc + SP_K * s);
        p.qb = load_words<NW>(xsrc + SP_K * s + 16);
        p.d = dsrc[2 * s];
    };
    issue(P0, 0);
    if (nst > 1) issue(P1, 1);

    // the token's power of two: 127 max_b d0[b] = f 2^e with f in [0.5, 1), s = 14 - e (clamped so that 2^s and
    // 2^-s stay normal floats); the TPR threads of a row split its blocks and meet by shuffles
    float up;
    {
        const float *drow = a.dx + xrow * nb;
        float m = 0.0f;
        for (int b = xp; b < nb; b += TPR) m = fmaxf(m, drow[b]);
#pragma unroll
        for (int o = 1; o < TPR; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        int ex = 0;
        if (m > 0.0f) (void)frexpf(127.0f * m, &ex);
        int sh = 14 - ex;
        sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
        up = ldexpf(1.0f, sh);
        if (xp == 0) sT[xr] = ldexpf(1.0f, -sh);
    }

    auto commit = [&](auto cc, const Pre &p) {
        constexpr int c = decltype(cc)::value;
        _Float16 *sw = pick2<c>(sW0, sW1), *sx = pick2<c>(sX0, sX1);
        uint16_t *sd = pick2<c>(sD0, sD1);
        S::decode(p.raw, lut, sw + (tid >> 1) * SP_ROW + 32 * wh);
        uint32_t o[VJ];
#pragma unroll
        for (int k = 0; k < NW; ++k) pairs_to_h2(p.qa.w[k], p.qb.w[k], o + 4 * k);
        uint4 *dst = (uint4 *)(sx + xr * SP_ROW + 32 * xb + 2 * j0);
#pragma unroll
        for (int k = 0; k < VJ / 4; ++k) dst[k] = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
        if (j0 == 0) sd[xr * 2 + xb] = __builtin_bit_cast(uint16_t, (_Float16)(p.d * up));
    };

    constexpr int RT = G::RT, CT = G::CT;
    const int wr0 = (wave / G::WC) * RT * 16, wc0 = (wave % G::WC) * CT * 16;
    f4 acc[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // the stage's MFMAs: per block, each token tile's hi and lo fragments, then its RT hi and RT lo products
    auto compute = [&](auto cc) {
        constexpr int c = decltype(cc)::value;
        const _Float16 *sw = pick2<c>(sW0, sW1), *sx = pick2<c>(sX0, sX1);
        const uint16_t *sd = pick2<c>(sD0, sD1);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int kk = 32 * b + 8 * (lane >> 4);
            h8 fa[RT];
#pragma unroll
            for (int i = 0; i < RT; ++i) fa[i] = *(const h8 *)(sw + (wr0 + 16 * i + (lane & 15)) * SP_ROW + kk);
#pragma unroll
            for (int j = 0; j < CT; ++j) {
                const int tr = wc0 + 16 * j + (lane & 15);
                const uint4 x = *(const uint4 *)(sx + tr * SP_ROW + kk);
                const uint32_t ds = sd[tr * 2 + b];
                const h2 dd = __builtin_bit_cast(h2, ds | (ds << 16));
                const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
                uint32_t hv[4], lv[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const h2 xv = __builtin_bit_cast(h2, xw[q]);
                    const h2 h = xv * dd;
                    hv[q] = __builtin_bit_cast(uint32_t, h);
                    lv[q] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(xv, dd, -h));
                }
                const h8 fh = __builtin_bit_cast(h8, make_uint4(hv[0], hv[1], hv[2], hv[3]));
                const h8 fl = __builtin_bit_cast(h8, make_uint4(lv[0], lv[1], lv[2], lv[3]));
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fh, acc[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fl, acc[i][j], 0, 0, 0);
            }
        }
    };

    // stage s (parity c) is in LDS buffer c and its register set is free: issue stage s + 2 into it, compute stage
    // s, commit stage s + 1 (register set 1 - c) into buffer 1 - c, whose stage s - 1 every wave finished before the
    // previous barrier
    auto step = [&](auto cc, int s) {
        constexpr int c = decltype(cc)::value;
        if (s + 2 < nst) issue(pick2<c>(P0, P1), s + 2);
        compute(cc);
        if (s + 1 < nst) commit(IC<1 - c>{}, pick2<1 - c>(P0, P1));
        __syncthreads();
    };

    __syncthreads();  // the table
    commit(IC<0>{}, P0);
    __syncthreads();
    for (int s = 0; s < nst; s += 2) {
        step(IC<0>{}, s);
        if (s + 1 < nst) step(IC<1>{}, s + 1);
    }

    // store: lane holds rows 4 (lane / 16) .. + 3 of each 16 x 16 tile, token column lane % 16
    const float sc = a.es ? a.es[e] : a.osc;
#pragma unroll
    for (int j = 0; j < CT; ++j) {
        const int tt = wc0 + 16 * j + (lane & 15);
        long long yrow;
        if constexpr (MOE) {
            if (tt >= tn) continue;
            yrow = (long long)orow[tt] * a.N;
        } else {
            const int t = tbase + tt;
            if (t >= a.T) continue;
            yrow = (long long)t * a.ldy;
        }
        const float f = sc * sT[tt];
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const int n = n0 + wr0 + 16 * i + 4 * (lane >> 4);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (n + r < a.N) a.y[yrow + n + r] = acc[i][j][r] * f;
        }
    }
}

template <int TYPE>
hipError_t launch_t(const GemmArgs &a, dim3 grid, hipStream_t stream) {
    if (a.n_tiles) hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T_SMALL, true>), grid, dim3(SP_THREADS), 0, stream, a);
    else if (a.tt == SP_T_SMALL)
        hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T_SMALL, false>), grid, dim3(SP_THREADS), 0, stream, a);
    else hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T, false>), grid, dim3(SP_THREADS), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

bool gemm_split(int type) { return type == TY_FP4 || type == TY_FAST || type == TY_NVFP4; }

int gemm_split_k_multiple() { return SP_K; }

int gemm_split_rows() { return SP_ROWS; }

int gemm_split_token_tile(bool moe, int T) { return moe || T <= SP_T_SMALL ? SP_T_SMALL : SP_T; }

hipError_t launch_gemm_split(int type, const GemmArgs &a, dim3 grid, hipStream_t stream) {
    switch (type) {
    case TY_FP4: return launch_t<TY_FP4>(a, grid, stream);
    case TY_FAST: return launch_t<TY_FAST>(a, grid, stream);
    case TY_NVFP4: return launch_t<TY_NVFP4>(a, grid, stream);
    default: return hipErrorInvalidDeviceFunction;
    }
}

}  // namespace pq
