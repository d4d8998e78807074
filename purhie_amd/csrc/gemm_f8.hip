// gemm_f8.hip -- the ROCmFP4 prefill GEMM done exactly on gfx950's f8f6f4 matrix core: a measured alternative
// to the split GEMM (gemm_split.hip), reachable through the test hook qmatvec_debug_gemm_f8f6f4 and the
// benchmark's --f8f6f4 leg, not through qmatvec_launch_q8_batch.
//
// The reference's prefill (src/matvec_q.hip:2566-2973) forms one exact integer dot per 16-value half of a ROCmFP4
// block and scales it by its UE4M3 half-scale and the token's block scale. On the f8f6f4 matrix core that integer
// is reachable, but only like this:
//   - weights: the Codebook10 levels {0, 1, 2, 3, 4, 6, 8, 10} with their signs are E4M3 values; the UE4M3 scale
//     cannot ride along (level times scale needs up to 7 significant bits, E4M3 holds 4; the instruction's own
//     block scales are E8M0 powers of two for 32 values, and ROCmFP4 scales each 16);
//   - activations: q0 (8 significant bits) enters as two E4M3 planes, 16 (q >> 4) in -128..112 and q & 15 in
//     0..15, both exact; two MFMAs into one accumulator give sum level * q exactly (|sum| < 2^24);
//   - a 32x32x64 instruction sums 64 K values, four 16-value groups with four different scale products, so each
//     group takes its own pair of instructions with the other 48 values of the weight operand zeroed;
//   - per group and output, one float step y += (e_w d_x) c on the vector unit: the reference's epilogue.
// Eight instructions per 64 values where the products need one: 8 times the useful work at the fp8 rate (5
// PFLOP/s), against the split GEMM's 2 times at the fp16 rate (2.5 PFLOP/s), so twice its matrix-core time, and the
// epilogue adds two vector instructions per output and group. The kernel is correct (its outputs are checked
// against the oracle within 1e-5 sum |w x|), staged as the other GEMMs are (LDS double-buffered, one barrier per
// 64-value stage, the next stage's loads in flight), and timed against the split GEMM.
//
// Workgroup: 256 threads (4 waves of 64 rows x 64 tokens: 2 x 2 tiles of 32 x 32), 128 weight rows x 128 tokens.
#include "device.h"
#include "kernels.h"

namespace pq {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int F8_ROWS = 128, F8_T = 128;

// LDS place of 16-byte chunk ch (0..3) of row r of a stage (64 fp8 values a row): chunk ch of the 16 rows of group
// r / 16 lie side by side, so the 16 lanes that read one chunk column of 16 rows touch 256 consecutive bytes, all
// 64 banks (gfx950 serves a 16-byte read 16 lanes a pass; rows of 80 bytes measured two passes a read)
__device__ __forceinline__ int f8_at(int r, int ch) { return ((r >> 4) << 10) + (ch << 8) + ((r & 15) << 4); }

// four FP4 codes (magnitude index 0..7 in each byte, sign 0x80) -> their E4M3 bytes: 0, 1, 2, 3 | 4, 6, 8, 10
__device__ __forceinline__ uint32_t cb_e4m3(uint32_t mag, uint32_t sign) {
    return __builtin_amdgcn_perm(0x52504C48u, 0x44403800u, mag) | sign;
}

// four 4-bit indices (one a byte) -> bytes of a 16-entry table (t0: entries 0..3, t1: 4..7, t2: 8..11, t3:
// 12..15)
__device__ __forceinline__ uint32_t lut16(uint32_t n, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, n & 0x07070707u);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, n & 0x07070707u);
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// four int8 values -> E4M3 bytes of 16 (q >> 4) and of q & 15
__device__ __forceinline__ void q_planes(uint32_t q, uint32_t &h, uint32_t &l) {
    h = lut16((q >> 4) & 0x0f0f0f0fu, 0x64605800u, 0x6e6c6a68u, 0xeaeceef0u, 0xd8e0e4e8u);
    l = lut16(q & 0x0f0f0f0fu, 0x44403800u, 0x4e4c4a48u, 0x53525150u, 0x57565554u);
}

__global__ void __launch_bounds__(256, 2) k_gemm_f8_exact(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][F8_ROWS * 64];
    __shared__ __attribute__((aligned(16))) uint8_t sBh[2][F8_T * 64], sBl[2][F8_T * 64];
    __shared__ __attribute__((aligned(16))) float sE[2][4][F8_ROWS];  // UE4M3 half-scale of (group, row)
    __shared__ __attribute__((aligned(16))) float sD[2][F8_T][2];     // d0 of (token, block)

    int tt, rt;
    xcd_tile(tt, rt, 4);
    const int tbase = tt * F8_T, n0 = rt * F8_ROWS;
    const int K = a.K, nb = K / 32, ns = K / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // staging roles: weight row sr = tid / 2, block sb = tid % 2 of the stage; token row sr, half sb
    const int sr = tid >> 1, sb = tid & 1;
    const int wrow_i = n0 + sr < a.N ? n0 + sr : a.N - 1;
    const uint8_t *wrow = a.W + (long long)wrow_i * a.row_bytes;
    const long long xrow = tbase + sr < a.T ? tbase + sr : a.T - 1;
    const int8_t *xsrc = a.xq + xrow * K + 32 * sb;
    const float *dsrc = a.dx + xrow * nb + sb;

    struct Pre {
        uint32_t w[5], off;
        uint4 q0, q1;
        float d;
    };
    auto issue = [&](Pre &p, int s) {
        s = s < ns ? s : ns - 1;
        const uint8_t *b = wrow + (long long)(2 * s + sb) * 18;
        p.off = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *al = b - p.off;
#pragma unroll
        for (int k = 0; k < 5; ++k) p.w[k] = ld32(al + 4 * k);
        p.q0 = *(const uint4 *)(xsrc + 64 * s);
        p.q1 = *(const uint4 *)(xsrc + 64 * s + 16);
        p.d = dsrc[2 * s];
    };
    auto commit = [&](int c, const Pre &p) {
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t w = align_bytes(p.w[k + 1], p.w[k], p.off);
            lo[k] = cb_e4m3(w & 0x07070707u, (w << 4) & 0x80808080u);
            hi[k] = cb_e4m3((w >> 4) & 0x07070707u, w & 0x80808080u);
        }
        *(uint4 *)(sA[c] + f8_at(sr, 2 * sb)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4 *)(sA[c] + f8_at(sr, 2 * sb + 1)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        const uint32_t sc = p.w[4] >> (8 * p.off);
        sE[c][2 * sb][sr] = ue4m3_half(sc);
        sE[c][2 * sb + 1][sr] = ue4m3_half(sc >> 8);
        const uint32_t qw[8] = {p.q0.x, p.q0.y, p.q0.z, p.q0.w, p.q1.x, p.q1.y, p.q1.z, p.q1.w};
        uint32_t h[8], l[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) q_planes(qw[k], h[k], l[k]);
        *(uint4 *)(sBh[c] + f8_at(sr, 2 * sb)) = make_uint4(h[0], h[1], h[2], h[3]);
        *(uint4 *)(sBh[c] + f8_at(sr, 2 * sb + 1)) = make_uint4(h[4], h[5], h[6], h[7]);
        *(uint4 *)(sBl[c] + f8_at(sr, 2 * sb)) = make_uint4(l[0], l[1], l[2], l[3]);
        *(uint4 *)(sBl[c] + f8_at(sr, 2 * sb + 1)) = make_uint4(l[4], l[5], l[6], l[7]);
        sD[c][sr][sb] = p.d;
    };

    // wave tile: rows wr0 .. + 63, tokens wc0 .. + 63; the 32 x 32 output layout: lane's token column lane % 32,
    // accumulator v at row 8 (v / 4) + 4 (lane / 32) + v % 4
    const int wr0 = (wave >> 1) * 64, wc0 = (wave & 1) * 64;
    const int half = lane >> 5;
    v16f y[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) y[i][j][v] = 0.0f;

    auto compute = [&](int c) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // lane's 32 weight bytes: row wr0 + 32 i + lane % 32, K values 32 half .. + 31 (groups 2 half, 2 half + 1)
            const int ra = wr0 + 32 * i + (lane & 31);
            const uint4 a0 = *(const uint4 *)(sA[c] + f8_at(ra, 2 * half));
            const uint4 a1 = *(const uint4 *)(sA[c] + f8_at(ra, 2 * half + 1));
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                // the weight operand of group g: its 16 values where they lie, zeros elsewhere
                const bool mine = half == (g >> 1);
                const uint4 src = (g & 1) ? a1 : a0;
                const uint4 keep = mine ? src : make_uint4(0u, 0u, 0u, 0u);
                v8i am;
                const uint4 z = make_uint4(0u, 0u, 0u, 0u);
                const uint4 lo = (g & 1) ? z : keep, hi = (g & 1) ? keep : z;
                am[0] = (int)lo.x; am[1] = (int)lo.y; am[2] = (int)lo.z; am[3] = (int)lo.w;
                am[4] = (int)hi.x; am[5] = (int)hi.y; am[6] = (int)hi.z; am[7] = (int)hi.w;
                float e[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 ev = *(const float4 *)(&sE[c][g][wr0 + 32 * i + 8 * q + 4 * half]);
                    e[4 * q] = ev.x;
                    e[4 * q + 1] = ev.y;
                    e[4 * q + 2] = ev.z;
                    e[4 * q + 3] = ev.w;
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int tr = wc0 + 32 * j + (lane & 31);
                    const uint4 h0 = *(const uint4 *)(sBh[c] + f8_at(tr, 2 * half));
                    const uint4 h1 = *(const uint4 *)(sBh[c] + f8_at(tr, 2 * half + 1));
                    const uint4 l0 = *(const uint4 *)(sBl[c] + f8_at(tr, 2 * half));
                    const uint4 l1 = *(const uint4 *)(sBl[c] + f8_at(tr, 2 * half + 1));
                    const v8i bh = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z,
                                    (int)h1.w};
                    const v8i bl = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z,
                                    (int)l1.w};
                    v16f cz = {};
                    v16f cg = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(am, bh, cz, 0, 0, 0, 127, 0, 127);
                    cg = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(am, bl, cg, 0, 0, 0, 127, 0, 127);
                    const float d = sD[c][tr][g >> 1];
#pragma unroll
                    for (int v = 0; v < 16; ++v) y[i][j][v] = fmaf(e[v] * d, cg[v], y[i][j][v]);
                }
            }
        }
    };

    Pre P;
    issue(P, 0);
    commit(0, P);
    issue(P, 1);
    __syncthreads();
    for (int s = 0; s < ns; ++s) {
        const int c = s & 1;
        commit(1 - c, P);  // stage s + 1 (loaded during stage s - 1's compute) into the idle buffer
        issue(P, s + 2);
        compute(c);
        __syncthreads();
    }

    const float sc = a.osc;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = tbase + wc0 + 32 * j + (lane & 31);
        if (t >= a.T) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wr0 + 32 * i + 8 * q + 4 * half;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (n + r < a.N) a.y[(long long)t * a.ldy + n + r] = y[i][j][4 * q + r] * sc;
            }
    }
}

}  // namespace

hipError_t launch_gemm_f8_exact(const GemmArgs &a, hipStream_t stream) {
    if (a.K % 64 != 0 || a.T <= 0 || a.N <= 0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.T + F8_T - 1) / F8_T), (unsigned)((a.N + F8_ROWS - 1) / F8_ROWS));
    hipLaunchKernelGGL(k_gemm_f8_exact, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace pq
