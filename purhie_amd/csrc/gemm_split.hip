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
// per block, as many VALU cycles as the block's MFMAs take; the second plane costs MFMA cycles instead. (Measured on
// gfx950: a wave's VALU instructions are free beside its MFMAs up to two per v_mfma_f32_16x16x32_f16; each further
// one costs about its own 4 cycles.)
//
// Workgroup: 256 threads (4 waves of 128 rows x TT / 2 tokens), two per CU, over 256 weight rows x TT tokens; K in
// stages of one 32-value block, double-buffered in LDS with one barrier per stage; every global load is issued PD
// stages before its LDS store (2 for the dense 128-token tiles, whose registers allow no more; 4 for the 64-token
// tiles: MoE expert tiles, prefill of config 4's sizes 339 -> 327 us). Staging per stage: thread t decodes block s of weight row n0 + t into fp16, and
// converts TT / 8 consecutive int8 values of one token row to fp16 integers, with the (token, block) scale ds.
// Each wave makes the hi and lo fragments of its token tiles and runs the MFMAs at raised wave priority, so that
// the other workgroup's staging on the same SIMD fills the VALU slots beside them.
#include "device.h"
#include "kernels.h"

namespace pq {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int SP_ROWS = 256;         // weight rows per workgroup, dense prompts of more than SP_T_SMALL tokens
constexpr int SP_ROWS_SMALL = 128;   // the same for MoE expert tiles and short prompts (twice the workgroups)
constexpr int SP_T = 128;            // tokens per workgroup, dense
constexpr int SP_T_SMALL = 64;       // MoE expert tiles (a few dozen entries on average) and prompts of <= 64 tokens

// LDS place (bytes) of 16-byte chunk ch (0..3, values 8 ch .. 8 ch + 7) of a stage's row r (32 fp16 values a row):
// chunk ch of the 16 rows of group r / 16 lie side by side, so a fragment read (lane: row 16 i + lane % 16, chunk
// lane / 16) touches 1 KiB as one contiguous read does, with no bank conflict; 80-byte padded rows took two LDS
// passes per fragment read (a probe kernel under rocprofv3, SQ_LDS_BANK_CONFLICT per instruction). The weight
// stores (a thread a row) are conflict-free too; the token stores of TPR threads a row keep the conflicts the
// padded rows had.
__device__ __forceinline__ int sp_at(int r, int ch) { return ((r >> 4) << 10) + (ch << 8) + ((r & 15) << 4); }
constexpr int SP_GROUP = 4;          // token tiles advancing together over the row tiles (XCD order)
constexpr int SP_PD = 2;             // prefetch distance (stages), dense 128-token tiles
constexpr int SP_PD_SMALL = 4;       // the same, dense 64-token tiles
constexpr int SP_PD_MOE = 4;         // the same, MoE expert tiles

// a workgroup of 256 threads (4 waves: 2 along the rows, 2 along the tokens, each RT x CT tiles of 16 x 16) over
// ROWS weight rows x TT tokens; per stage, PW staging threads decode a row's block (each 4 / PW of its code words)
// and VN token values go to each thread, TPR threads a token row
template <int TT, int ROWS>
struct SpGeo {
    static constexpr int RT = ROWS / 32, CT = TT / 32;
    static constexpr int PW = 256 / ROWS;
    static constexpr int VN = TT / 8;
    static constexpr int TPR = 32 / VN;
    static_assert((ROWS == 256 || ROWS == 128) && (TT == 128 || TT == 64), "tile geometry");
};

// Four FP4 codes in the low nibbles of w and four in the high nibbles, as fp16 values times their scales, two
// half2 each (lo: the low nibbles' values in byte order, scaled by slo; hi: the high nibbles', by shi). The codebook's
// fp16 values have a zero low byte, so v_perm_b32 looks the high bytes of four magnitudes up in an 8-byte table
// (TOP 10: ROCmFP4's levels {0, 1, 2, 3, 4, 6, 8, 10}; TOP 12: E2M1 doubled), the sign bits are or-ed in, two more
// byte selections make the half2, and a packed fp16 multiply applies the scale (exact: a level times a UE4M3
// half-scale value has at most 8 significant bits). (v_cvt_scalef32_pk_f16_fp8 would fold the scale in, but it applies
// only the scale's power of two.)
template <int TOP>
__device__ __forceinline__ void fp4_word(uint32_t w, h2 slo, h2 shi, uint32_t lo[2], uint32_t hi[2]) {
    constexpr uint32_t TLO = 0x42403c00u, THI = TOP == 10 ? 0x49484644u : 0x4a484644u;
    const uint32_t ml = __builtin_amdgcn_perm(THI, TLO, w & 0x07070707u) | ((w << 4) & 0x80808080u);
    const uint32_t mh = __builtin_amdgcn_perm(THI, TLO, (w >> 4) & 0x07070707u) | (w & 0x80808080u);
    auto h = [](uint32_t m, uint32_t sel, h2 sc) {
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(0u, m, sel)) * sc);
    };
    lo[0] = h(ml, 0x010c000cu, slo);
    lo[1] = h(ml, 0x030c020cu, slo);
    hi[0] = h(mh, 0x010c000cu, shi);
    hi[1] = h(mh, 0x030c020cu, shi);
}

__device__ __forceinline__ h2 h2of(float v) {
    h2 r;
    r.x = (_Float16)v;  // exact: a UE4M3 half-scale value is an fp16 value
    r.y = r.x;
    return r;
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
    // 32-value block kb of the row: five words from the 4-aligned address at or below it (they end at most 3 bytes
    // past the block, inside the 4-aligned word that holds its last byte)
    __device__ static void load(const uint8_t *row, int kb, Raw &r) {
        const uint8_t *b = row + (long long)kb * BB;
        r.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *al = b - r.off;
#pragma unroll
        for (int k = 0; k < 5; ++k) r.w[k] = ld32(al + 4 * k);
    }
    // byte i of the codes holds values i (low nibble, scale e0) and i + 16 (high, scale e1). Part p of P decodes
    // code words 4 p / P .. (word k: values 4k .. 4k + 3 and 16 + 4k .. 16 + 4k + 3) into LDS row `row` of sw, the
    // block's 32 values in order.
    template <int P>
    __device__ static void decode(const Raw &r, _Float16 *sw, int row, int p) {
        uint8_t *base = (uint8_t *)sw;
        const uint32_t sc = r.w[4] >> (8 * r.off);  // the scale bytes at block offset 16 (and 17)
        const h2 e0 = h2of(ue4m3_half(sc));
        const h2 e1 = TYPE == TY_FP4 ? h2of(ue4m3_half(sc >> 8)) : e0;
#pragma unroll
        for (int k = 0; k < 4 / P; k += 2) {
            const int k0 = 4 / P * p + k;
            uint32_t lo[2][2], hi[2][2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                fp4_word<TOP>(align_bytes(r.w[k0 + j + 1], r.w[k0 + j], r.off), e0, e1, lo[j], hi[j]);
            *(uint4 *)(base + sp_at(row, k0 >> 1)) = make_uint4(lo[0][0], lo[0][1], lo[1][0], lo[1][1]);
            *(uint4 *)(base + sp_at(row, 2 + (k0 >> 1))) = make_uint4(hi[0][0], hi[0][1], hi[1][0], hi[1][1]);
        }
    }
};

// NVFP4: 36-byte blocks of 64 values (4 UE4M3 scale bytes, then four 16-value sub-blocks of 8 bytes, byte i: values
// i low, 8 + i high). 32-value block kb is half h = kb & 1 (sub-blocks 2h, 2h + 1, each with its scale) of block
// kb / 2.
template <>
struct SpW<TY_NVFP4> {
    static constexpr int TOP = 12;
    struct Raw {
        uint32_t sc, v[4];
    };
    __device__ static void load(const uint8_t *row, int kb, Raw &r) {
        const int h = kb & 1;
        const uint8_t *b = row + (long long)(kb >> 1) * 36;
        r.sc = ld32(b) >> (16 * h);
#pragma unroll
        for (int k = 0; k < 4; ++k) r.v[k] = ld32(b + 4 + 16 * h + 4 * k);
    }
    // sub-block q (code words 2q, 2q + 1; word k: values 4k' .. 4k' + 3 low nibbles, 8 + 4k' .. high, k' = k & 1)
    // with its own scale; part p of P decodes sub-blocks 2 p / P ..
    template <int P>
    __device__ static void decode(const Raw &r, _Float16 *sw, int row, int p) {
        uint8_t *base = (uint8_t *)sw;
#pragma unroll
        for (int k = 0; k < 4 / P; k += 2) {
            const int k0 = 4 / P * p + k, q = k0 >> 1;
            const h2 e = h2of(nv_scale(r.sc >> (8 * q)));
            uint32_t lo[2][2], hi[2][2];
#pragma unroll
            for (int j = 0; j < 2; ++j) fp4_word<TOP>(r.v[k0 + j], e, e, lo[j], hi[j]);
            *(uint4 *)(base + sp_at(row, 2 * q)) = make_uint4(lo[0][0], lo[0][1], lo[1][0], lo[1][1]);
            *(uint4 *)(base + sp_at(row, 2 * q + 1)) = make_uint4(hi[0][0], hi[0][1], hi[1][0], hi[1][1]);
        }
    }
};

// four int8 values (a word) as two fp16 pairs in order: the byte b ^ 0x80 under 0x64 is the fp16 1024 + 128 + b,
// minus 1152
__device__ __forceinline__ void i8_to_h2(uint32_t a, uint32_t *o) {
    h2 bias;
    bias.x = (_Float16)1152.0f;
    bias.y = (_Float16)1152.0f;
    const uint32_t w0 = __builtin_amdgcn_perm(0u, a, 0x0c010c00u) ^ 0x64806480u;
    const uint32_t w1 = __builtin_amdgcn_perm(0u, a, 0x0c030c02u) ^ 0x64806480u;
    o[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w0) - bias);
    o[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w1) - bias);
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
    } else {
        static_assert(N == 2, "8 or 16 bytes");
        const uint2 v = *(const uint2 *)p;
        r.w[0] = v.x;
        r.w[1] = v.y;
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

// The SwiGLU pair's epilogue. The up waves (2, 3) put u = acc sc_u 2^-s into sU (their token half, [token][129]
// floats, within the LDS weight buffer the finished loop no longer reads); after a barrier each gate wave (0, 1) takes
// g = acc sc_g 2^-s of the same (row, token), v = g / (1 + exp(-g)) u (the arithmetic of gpu_swiglu), and quantizes
// each 32-row block of a token as the activation quantizer does: am = max |v| over the block (8 values in each of the
// 4 lanes of the token's column), q = rint(v 127 / am), d = fp16(am / 127), s0 = fp16(d sum q). The lane's 4
// consecutive rows of a tile are 4 consecutive bytes of q. Output row of entry j: out_rows[j]; padding entries store
// nothing.
template <int RT, int CT>
__device__ __forceinline__ void swiglu_epilogue(const GemmArgs &a, const f4 (&acc)[RT][CT], int e, int n0, int tn,
                                                const int32_t *orow, const float *sT, float *sU, int wave, int lane) {
    static_assert(RT == 8, "128 rows a wave: four 32-row blocks");
    constexpr int UP = 129;
    if (wave >= 2) {
        const float sc = a.es2 ? a.es2[e] : a.osc2;
#pragma unroll
        for (int j = 0; j < CT; ++j) {
            const int tl = 16 * j + (lane & 15), tt = 16 * CT * (wave & 1) + tl;
            const float f = sc * sT[tt];
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) sU[tl * UP + 16 * i + 4 * (lane >> 4) + r] = acc[i][j][r] * f;
        }
    }
    __syncthreads();
    if (wave >= 2) return;
    const float sc = a.es ? a.es[e] : a.osc;
    const int N = a.N;
#pragma unroll
    for (int j = 0; j < CT; ++j) {
        const int tl = 16 * j + (lane & 15), tt = 16 * CT * (wave & 1) + tl;
        const bool store = tt < tn;
        const long long hrow = store ? (long long)orow[tt] : 0;
        const float f = sc * sT[tt];
#pragma unroll
        for (int b = 0; b < RT / 2; ++b) {
            float v[8];
            float am = 0.0f;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * (2 * b + h) + 4 * (lane >> 4) + r;
                    const float g = acc[2 * b + h][j][r] * f, u = sU[tl * UP + row];
                    v[4 * h + r] = g / (1.0f + expf(-g)) * u;
                    am = fmaxf(am, fabsf(v[4 * h + r]));
                }
            am = fmaxf(am, __shfl_xor(am, 16, 64));
            am = fmaxf(am, __shfl_xor(am, 32, 64));
            const float id0 = am != 0.0f ? 127.0f / am : 0.0f;
            uint32_t qw[2] = {0u, 0u};
            int qs = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int q = (int)rintf(v[k] * id0);
                qs += q;
                qw[k >> 2] |= (uint32_t)(q & 0xff) << (8 * (k & 3));
            }
            qs += __shfl_xor(qs, 16, 64);
            qs += __shfl_xor(qs, 32, 64);
            if (store) {
                int8_t *q0 = a.hq + hrow * N + n0 + 32 * b + 4 * (lane >> 4);
                *(uint32_t *)q0 = qw[0];
                *(uint32_t *)(q0 + 16) = qw[1];
                if ((lane >> 4) == 0) {
                    const float d = am / 127.0f;
                    const long long bi = hrow * (N / 32) + (n0 + 32 * b) / 32;
                    a.hd[bi] = __half2float(__float2half(d));
                    if (a.hs) {
                        float p = d * (float)qs;
                        __asm__ volatile("" : "+v"(p));  // (fp16 of the fp32 product, as the quantizer)
                        a.hs[bi] = __float_as_int(__half2float(__float2half(p)));
                    }
                }
            }
        }
    }
}

// capture mode: four ints at cap[i] (dropped past cap_n)
__device__ __forceinline__ void cap_put4(const GemmArgs &a, long long i, uint4 v) {
    if (i >= 0 && i + 4 <= a.cap_n) *(uint4 *)(a.cap + i) = v;
}

// PD: the prefetch distance in stages (2 or 4): stage s's global loads are issued PD stages before its LDS store,
// into one of PD register sets. SWP (MoE, the gate / up pair): the workgroup's rows are rows n0 .. n0 + ROWS / 2 - 1
// of W (gate, waves 0 and 1) and the same rows of W2 (up, waves 2 and 3), and the epilogue writes
// SwiGLU(gate, up) = g / (1 + exp(-g)) u quantized to Q8_0 (hq, hd, hs) instead of the two outputs. CAP (capture
// mode, a test hook): the same kernel, which also stores the operands it hands the matrix core (each staged weight
// block, each token's hi and lo fragments and its power of two) at gemm_split_capture_layout.
template <int TYPE, int TT, int ROWS, bool MOE, int PD, bool SWP = false, bool CAP = false>
__global__ void __launch_bounds__(256, ROWS == SP_ROWS_SMALL ? 3 : 2) k_gemm_split(GemmArgs a) {
    static_assert(PD == 2 || PD == 4, "prefetch distance");
    static_assert(!SWP || (MOE && ROWS == 256 && TT == 64), "the SwiGLU pair: MoE tiles of 256 rows x 64 tokens");
    static_assert(!(SWP && CAP), "no capture of the SwiGLU pair");
    using S = SpW<TYPE>;
    using G = SpGeo<TT, ROWS>;
    constexpr int PW = G::PW;
    constexpr int VN = G::VN, TPR = G::TPR, NW = VN / 4;
    // (the SwiGLU epilogue reuses sW0 / sW1 as [32][129] floats each)
    constexpr int WH = SWP ? (ROWS * 32 > 2 * 32 * 129 ? ROWS * 32 : 2 * 32 * 129) : ROWS * 32;
    __shared__ __attribute__((aligned(16))) _Float16 sW0[WH], sW1[WH];
    __shared__ __attribute__((aligned(16))) _Float16 sX0[TT * 32], sX1[TT * 32];
    __shared__ uint16_t sD0[TT], sD1[TT];  // ds of (token, the stage's block), fp16 bits
    __shared__ float sT[TT];               // 2^-s per token

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
        n0 = SWP ? (int)blockIdx.x * (ROWS / 2) : moe_row_tile(a) * ROWS;
    } else {  // grid (token tiles, row tiles), renumbered XCD by XCD
        int tt, rt;
        xcd_tile(tt, rt, SP_GROUP);
        tbase = tt * TT;
        n0 = rt * ROWS;
    }
    // token row of tile position j: real rows for j < n (dense: < T), else a repeat of a valid row whose outputs are
    // not stored
    auto trow = [&](int j) -> long long {
        if constexpr (MOE) return rows[j < tn ? j : 0];
        const int t = tbase + j;
        return t < a.T ? t : a.T - 1;
    };

    const int K = a.K, nb = K / 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // staging roles. Weights: LDS row lr = tid / PW (global row n0 + lr; SWP: rows 0 .. ROWS / 2 - 1 of W, then
    // of W2), part tid % PW of its block (rows past the end repeat the last; their outputs are not stored).
    // Tokens: row xr = tid / TPR, values x0 .. x0 + VN - 1 of each block. (Rows by tid % ROWS and tid % TT instead,
    // with conflict-free token stores, made the compiler wait for every load in flight each stage: 832 -> 1228 us.)
    const int lr = tid / PW, wp = tid % PW;
    const int wr = n0 + (SWP ? lr % (ROWS / 2) : lr);
    const uint8_t *wrow = (SWP && lr >= ROWS / 2 ? a.W2 : a.W) +
                          ((long long)e * a.N + (wr < a.N ? wr : a.N - 1)) * a.row_bytes;
    const int xr = tid / TPR, xp = tid % TPR, x0 = VN * xp;
    const long long xrow = trow(xr);
    const int8_t *xsrc = a.xq + xrow * K + x0;
    const float *dsrc = a.dx + xrow * nb;

    struct Pre {
        typename S::Raw raw;
        Words<NW> q;
        float d;
    };
    Pre P[PD];
    // stage s's loads; a stage past the end loads the last one again (the steady loop has no conditions: those
    // copies are committed into the idle LDS buffer after the last compute and never read)
    auto issue = [&](Pre &p, int s) {
        s = s < nb ? s : nb - 1;
        S::load(wrow, s, p.raw);
        p.q = load_words<NW>(xsrc + 32 * s);
        p.d = dsrc[s];  // (every thread of the row: no branch in the loop)
    };
#pragma unroll
    for (int i = 0; i < PD; ++i) issue(P[i], i);

    // the token's power of two: 127 max_b d0[b] = f 2^e with f in [0.5, 1), s = 14 - e (clamped so that 2^s and
    // 2^-s stay normal floats); the TPR threads of a row split its blocks and meet by shuffles
    float up;
    {
        const float *drow = a.dx + xrow * nb;
        float m = 0.0f;
        // sixteen loads in flight at a time (a loop of one load each waited for every load before it: the dense
        // 128-token tiles' 80 scales a thread were 80 memory round trips)
        constexpr int ML = 16;
        for (int b0 = xp; b0 < nb; b0 += ML * TPR) {
            float v[ML];
#pragma unroll
            for (int k = 0; k < ML; ++k) v[k] = b0 + k * TPR < nb ? drow[b0 + k * TPR] : 0.0f;
#pragma unroll
            for (int k = 0; k < ML; ++k) m = fmaxf(m, v[k]);
        }
#pragma unroll
        for (int o = 1; o < TPR; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        int ex = 0;
        if (m > 0.0f) (void)frexpf(127.0f * m, &ex);
        int sh = 14 - ex;
        sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
        up = ldexpf(1.0f, sh);
        if (xp == 0) sT[xr] = ldexpf(1.0f, -sh);
        if constexpr (CAP) {  // (row tile 0: every row tile forms the same)
            const bool live = MOE ? xr < tn : tbase + xr < a.T;
            if (xp == 0 && n0 == 0 && live)
                a.cap[gemm_split_capture_layout(K, a.cap_xr).s_off + xrow] = sh;
        }
    }

    auto commit = [&](auto cc, const Pre &p) {
        constexpr int c = decltype(cc)::value;
        _Float16 *sw = pick2<c>(sW0, sW1), *sx = pick2<c>(sX0, sX1);
        uint16_t *sd = pick2<c>(sD0, sD1);
        S::template decode<PW>(p.raw, sw, lr, wp);
        uint32_t o[VN / 2];
#pragma unroll
        for (int k = 0; k < NW; ++k) i8_to_h2(p.q.w[k], o + 2 * k);
#pragma unroll
        for (int k = 0; k < VN / 8; ++k)
            *(uint4 *)((uint8_t *)sx + sp_at(xr, x0 / 8 + k)) = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2],
                                                                           o[4 * k + 3]);
        sd[xr] = __builtin_bit_cast(uint16_t, (_Float16)(p.d * up));  // (the row's TPR threads: one value)
    };

    constexpr int RT = G::RT, CT = G::CT;
    const int wr0 = (wave >> 1) * RT * 16, wc0 = (wave & 1) * CT * 16;
    f4 acc[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // the stage's MFMAs: each token tile's hi and lo fragments, then its RT hi and RT lo products (stage index st:
    // the capture's)
    auto compute = [&](auto cc, int st) {
        constexpr int c = decltype(cc)::value;
        const _Float16 *sw = pick2<c>(sW0, sW1), *sx = pick2<c>(sX0, sX1);
        const uint16_t *sd = pick2<c>(sD0, sD1);
        if constexpr (CAP) {  // the weight row this thread staged (dense: token tile 0 only; expert tiles: each)
            if (wp == 0 && wr < a.N && (MOE || tbase == 0)) {
                const long long o = gemm_split_capture_layout(K, a.cap_xr).w_off +
                                    (((long long)e * a.N + wr) * nb + st) * 16;
#pragma unroll
                for (int q = 0; q < 4; ++q) cap_put4(a, o + 4 * q, *(const uint4 *)((const uint8_t *)sw + sp_at(lr, q)));
            }
        }
        {
            const int kk = 8 * (lane >> 4);
            h8 fa[RT];
#pragma unroll
            for (int i = 0; i < RT; ++i)
                fa[i] = *(const h8 *)((const uint8_t *)sw + sp_at(wr0 + 16 * i + (lane & 15), lane >> 4));
#pragma unroll
            for (int j = 0; j < CT; ++j) {
                const int tr = wc0 + 16 * j + (lane & 15);
                const uint4 x = *(const uint4 *)((const uint8_t *)sx + sp_at(tr, lane >> 4));
                const uint32_t ds = sd[tr];
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
                if constexpr (CAP) {  // the token's fragments (waves 0 and 1 of row tile 0)
                    if ((wave >> 1) == 0 && n0 == 0 && (MOE ? tr < tn : tbase + tr < a.T)) {
                        const long long o = (trow(tr) * nb + st) * 16 + kk / 2;
                        cap_put4(a, o, make_uint4(hv[0], hv[1], hv[2], hv[3]));
                        cap_put4(a, gemm_split_capture_layout(K, a.cap_xr).lo_off + o,
                                 make_uint4(lv[0], lv[1], lv[2], lv[3]));
                    }
                }
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fh, acc[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fl, acc[i][j], 0, 0, 0);
            }
        }
    };

    // step s (s = s0 + u, s0 a multiple of the unroll U, itself a multiple of PD): stage s is in LDS buffer s & 1
    // and its register set s % PD is free (committed by step s - 1). Commit stage s + 1 (register set (s + 1) % PD)
    // into buffer 1 - (s & 1), whose stage s - 1 every wave finished before the previous barrier; issue stage
    // s + PD into set s % PD; compute stage s. The steady loop has no conditions, so that the staging work (decode,
    // LDS stores, global loads) and the MFMAs of a step share one basic block and can be interleaved.
    constexpr int U = PD;
    auto step = [&](auto uu, int s0) {
        constexpr int u = decltype(uu)::value, c = u & 1;
        commit(IC<1 - c>{}, P[(u + 1) % PD]);
        issue(P[u % PD], s0 + u + PD);
        __builtin_amdgcn_sched_barrier(0);  // (measured: the staging ahead of the MFMAs, not mixed in, is faster)
        __builtin_amdgcn_s_setprio(1);      // the MFMA phase ahead of the other workgroup's staging on this SIMD
        compute(IC<c>{}, s0 + u);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
    };

    commit(IC<0>{}, P[0]);
    __syncthreads();
    // the stage count nb is even (the host's K multiple is 64): groups of U steps, then (U = 4) one pair
    int s = 0;
    for (; s + U <= nb; s += U) {
        step(IC<0>{}, s);
        step(IC<1>{}, s);
        if constexpr (U == 4) {
            step(IC<2>{}, s);
            step(IC<3>{}, s);
        }
    }
    if (U == 4 && s < nb) {
        step(IC<0>{}, s);
        step(IC<1>{}, s);
    }

    if constexpr (SWP) {
        swiglu_epilogue<RT, CT>(a, acc, e, n0, tn, orow, sT, (float *)(wave & 1 ? sW1 : sW0), wave, lane);
        return;
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
    if (a.n_tiles && a.hq)
        hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T_SMALL, SP_ROWS, true, SP_PD_MOE, true>), grid, dim3(256), 0, stream,
                           a);
    else if (a.cap && a.n_tiles)
        hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T_SMALL, SP_ROWS, true, SP_PD_MOE, false, true>), grid, dim3(256), 0,
                           stream, a);
    else if (a.cap && a.tt == SP_T_SMALL)
        hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T_SMALL, SP_ROWS_SMALL, false, SP_PD_SMALL, false, true>), grid,
                           dim3(256), 0, stream, a);
    else if (a.cap)
        hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T, SP_ROWS, false, SP_PD, false, true>), grid, dim3(256), 0, stream,
                           a);
    else if (a.n_tiles)
        hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T_SMALL, SP_ROWS, true, SP_PD_MOE>), grid, dim3(256), 0, stream, a);
    else if (a.tt == SP_T_SMALL)
        hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T_SMALL, SP_ROWS_SMALL, false, SP_PD_SMALL>), grid, dim3(256), 0,
                           stream, a);
    else hipLaunchKernelGGL((k_gemm_split<TYPE, SP_T, SP_ROWS, false, SP_PD>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

bool gemm_split(int type) { return type == TY_FP4 || type == TY_FAST || type == TY_NVFP4; }

int gemm_split_k_multiple() { return 64; }

int gemm_split_rows(bool moe, int T) { return !moe && T <= SP_T_SMALL ? SP_ROWS_SMALL : SP_ROWS; }

int gemm_split_token_tile(bool moe, int T) { return moe || T <= SP_T_SMALL ? SP_T_SMALL : SP_T; }

int gemm_split_swiglu_rows() { return SP_ROWS / 2; }

hipError_t launch_gemm_split(int type, const GemmArgs &a, dim3 grid, hipStream_t stream) {
    switch (type) {
    case TY_FP4: return launch_t<TY_FP4>(a, grid, stream);
    case TY_FAST: return launch_t<TY_FAST>(a, grid, stream);
    case TY_NVFP4: return launch_t<TY_NVFP4>(a, grid, stream);
    default: return hipErrorInvalidDeviceFunction;
    }
}

}  // namespace pq
