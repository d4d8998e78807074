// kernels.h -- internal launch interface between the C-ABI host layer (qmatvec.cpp, ...) and the HIP
// kernels of libpurhie_qmv. Not installed: the public interface is include/*.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pq {

// ggml type ids of the path's weight formats
constexpr int TY_Q8_0 = 8, TY_Q4_K = 12, TY_Q5_K = 13, TY_Q6_K = 14, TY_IQ4_XS = 23, TY_MXFP4 = 39, TY_NVFP4 = 40,
              TY_FP4 = 100, TY_FAST = 101;

// quantized activation output pointers (the layout of qmatvec_q8)
struct Q8Ptrs {
    int8_t *q0;
    float *d0;
    int8_t *qK;
    float *dK;
    int32_t *bsK;
    int32_t *s0;
};

hipError_t launch_quantize_q8(const float *x, int n, const Q8Ptrs &o, hipStream_t stream);

// Decode matvec over up to 4 stacked matrices of one type and K, T (1..4) tokens. Rows [bound[i-1],
// bound[i]) of the launch come from W[i] and go to y[i] (token t at y[i] + t * ystride[i]).
struct MvArgs {
    const uint8_t *W[4];
    float *y[4];
    int bound[4];
    long long ystride[4];
    float osc[4];
    long long row_bytes;
    const int8_t *q;     // token 0's quantized activation (Q8_0 or Q8_K values); token t at q + t * K
    const float *d;      // its scales; token t at d + t * (K / act block)
    const int32_t *bs;   // Q8_K group sums (K-quants); token t at bs + t * (K / 16)
    int Nt, K, L, T;
    int32_t *cap;        // capture mode (null: off): every scale group's integer dot is added into
                         // cap[(t * Nt + row) * (K / G) + group] (G = cap_group(type)); the buffer starts at zero
    // set (ROCmFP4_FAST, one token, K <= 1024): the activation is SiLU(lr_lo[i] lr_scale) for i < lr_n, 0 up to K,
    // quantized to Q8_0 in the kernel (q / d unused)
    const float *lr_lo;
    int lr_n;
    float lr_scale;
};
hipError_t launch_matvec(int type, const MvArgs &a, hipStream_t stream);
// the low-rank input (MvArgs lr_lo set): the tile kernel where it takes the shape, else the per-wave kernel, each
// with the activation made in the kernel as the launch_matvec of SwiGLU(lo scale, 1)'s quantization would see it
hipError_t launch_matvec_lr(int type, const MvArgs &a, hipStream_t stream);
constexpr int LR_MAXK = 1024;

// the values one weight scale covers (the capture's group): 16 for ROCmFP4, NVFP4 and Q6_K, else 32
constexpr int cap_group(int type) { return type == 100 || type == 40 || type == 14 ? 16 : 32; }

// MoE expert-indexed matvec (decode): grid (row groups, n_used * nmat, T)
struct MvIdArgs {
    const uint8_t *W[2];   // stacked experts of the first and second matrix
    const uint8_t *Wx[2];  // the matrices an id of -1 selects
    float *y[2];
    const float *es[2];    // per-expert output scales (null: s[m])
    float s[2], sx[2];
    long long row_bytes;
    const int32_t *ids;
    const int8_t *q;
    const float *d;
    const int32_t *bs;
    int n_used, x_per_slot, N, K, L, nmat, T;
    // tiles mode (n_tiles set; nmat 1, grid.y = entry i of a tile, grid.z = tile k): entry i of tile k (i <
    // tile_n[k]) multiplies input row in_rows[tile_start[k] + i] by expert tile_e[k] into output row out_rows[..]
    const int32_t *n_tiles, *tile_e, *tile_start, *tile_n, *in_rows, *out_rows;
    int tile, max_tiles;
    // set: the input rows are SwiGLU(sw_g, sw_u) (row in_row of each, K floats), quantized to Q8_0 in the kernel
    // (q / d unused; the tile kernel of a Q8_0-activation type only)
    const float *sw_g, *sw_u;
    // capture mode (null: off): the dots of entry (matrix m, output row o) go to
    // cap[((m * cap_rows + o) * N + row) * (K / G) + group] (cap_rows: T * n_used, or 0 in tiles mode)
    int32_t *cap;
    long long cap_rows;
    // routing in the launch (route_logits set; tile kernel, 256-thread tiles, route_ne <= 256, no tiles mode):
    // every workgroup routes its token from route_logits [T][route_ne] as the router kernel does, and the first
    // workgroup of each token writes its ids and weights to route_ids / route_wts [T][n_used] (ids is unused)
    const float *route_logits;
    int route_ne;
    int32_t *route_ids;
    float *route_wts;
};
hipError_t launch_matvec_id(int type, const MvIdArgs &a, hipStream_t stream);
bool matvec_id_swiglu_supported(int type, int K);

// the one-unit-per-lane tile kernels (mv_tile.hip); hipErrorNotSupported for a shape or alignment they do
// not take (launch_matvec / launch_matvec_id then use the per-wave kernels)
hipError_t launch_matvec_tile(int type, const MvArgs &a, hipStream_t stream);
hipError_t launch_matvec_tile_lr(int type, const MvArgs &a, hipStream_t stream);
hipError_t launch_matvec_id_tile(int type, const MvIdArgs &a, hipStream_t stream);

// per-scale-group integer dots (test hook)
hipError_t launch_block_dots(int type, const uint8_t *W, long long row_bytes, const int8_t *q, int32_t *out, int N,
                             int K, hipStream_t stream);

// Prefill GEMM over the quantized activation, read in place: dense tiles (n_tiles null) or MoE expert tiles.
struct GemmArgs {
    const uint8_t *W;       // dense: the matrix; MoE: stacked experts
    long long row_bytes;
    const int8_t *xq;       // int8 activation rows [rows][K]: Q8_K's qK for the K-quants, Q8_0's q0 otherwise
    const float *dx;        // their scales: dK [rows][K / 256] or d0 [rows][K / 32]
    const int32_t *xsum;    // K-quants: the Q8_K 16-value sums [rows][K / 16]
    float *y;
    long long ldy;
    int N, K, T;
    float osc;
    // MoE tiles (n_tiles null: dense)
    const int32_t *n_tiles, *tile_e, *tile_start, *tile_n, *in_rows, *out_rows;
    const float *es;        // per-expert output scales (null: osc)
    // MoE pair (W2 non-null): a second matrix of the same shape over the same tiles (the experts' gate and up) in
    // one grid: row-tile columns 0 .. rt - 1 are W's, rt .. 2 rt - 1 are W2's (output y2, scales es2 / osc2)
    const uint8_t *W2;
    float *y2;
    const float *es2;
    float osc2;
    int rt;
    // MoE pair with SwiGLU (hq set; split GEMM): the entries' SwiGLU(y, y2) rows quantized to Q8_0 instead of y and
    // y2: values hq [rows][N], scales hd [rows][N / 32], block sums hs (null: not written)
    int8_t *hq;
    float *hd;
    int32_t *hs;
    int tt;                 // split GEMM, dense: tokens per workgroup (gemm_split_token_tile); int8 GEMMs, MoE: the
                            // caller's tile (at most 64: the 64-token form)
    // capture mode (null: off; the integer-exact GEMMs): the exact integer each epilogue scales, per token (dense:
    // t; tiles: the entry's output row) and weight row: cap[(t * N + row) * (K / U) + unit], U = gemm_cap_unit(type)
    int32_t *cap;
    // the split GEMM's capture (cap set): its operands instead of integer sums, in cap_n ints (writes past them are
    // dropped) for activations of cap_xr rows; layout at gemm_split_capture_layout
    long long cap_n;
    int cap_xr;
};

// a MoE GEMM workgroup's row-tile column (blockIdx.x), with a switched to the pair's second matrix when the column
// lies in its half of the grid
__device__ inline int moe_row_tile(GemmArgs &a) {
    int bx = blockIdx.x;
    if (a.W2 && bx >= a.rt) {
        bx -= a.rt;
        a.W = a.W2;
        a.y = a.y2;
        a.es = a.es2;
        a.osc = a.osc2;
    }
    return bx;
}

int gemm_supported(int type);
// values per integer the type's GEMM exposes in capture mode (0: its sums are not integers, none captured)
int gemm_cap_unit(int type);
// the split-activation GEMM (gemm_split.hip: ROCmFP4, ROCmFP4_FAST, NVFP4; Q8_0 activation, xq = q0, dx = d0):
// dense grid (tokens / gemm_split_token_tile(false, T), rows / gemm_split_rows(false, T)), MoE grid (rows /
// gemm_split_rows(true, 0), tiles) with tiles of up to gemm_split_token_tile(true, 0) entries; K a multiple of
// gemm_split_k_multiple()
bool gemm_split(int type);
int gemm_split_k_multiple();
int gemm_split_rows(bool moe, int T);  // weight rows per workgroup
int gemm_split_token_tile(bool moe, int T);
// the MoE gate / up pair with SwiGLU (GemmArgs hq set): rows of each matrix per workgroup, grid (N / this, tiles)
int gemm_split_swiglu_rows();
hipError_t launch_gemm_split(int type, const GemmArgs &a, dim3 grid, hipStream_t stream);
// the exact ROCmFP4 GEMM on the f8f6f4 matrix core (gemm_f8.hip; a measured alternative, test hook only): dense,
// Q8_0 activation (xq = q0, dx = d0), K a multiple of 64
hipError_t launch_gemm_f8_exact(const GemmArgs &a, hipStream_t stream);
// The split GEMM's capture (GemmArgs cap set), in int32 units, nb = K / 32, XR = cap_xr activation rows: for
// activation row x and stage (32-value block) s, the fp16 hi plane at cap[(x * nb + s) * 16 ..] (32 halves in K
// order), the lo plane at lo_off + the same, the row's power of two s_x (the GEMM scales X by 2^s_x) at
// cap[s_off + x]; for weight row w (dense: the row; expert tiles: e * N + row), the 32 fp16 values it staged for
// block s at cap[w_off + (w * nb + s) * 16 ..]
struct SplitCapLayout {
    long long lo_off, s_off, w_off;
};
__host__ __device__ inline SplitCapLayout gemm_split_capture_layout(int K, int XR) {
    const long long plane = (long long)XR * (K / 32) * 16;
    return SplitCapLayout{plane, 2 * plane, 2 * plane + (XR + 3) / 4 * 4};
}

// CUs of the current device (read once per device; 256 when the query fails)
int device_cus();

// Float activations over F32 / F16 / BF16 weights (type ids 0, 1, 30): the decode matvec for T tokens (round:
// the activations rounded to the 16-bit weight type), the F16 / BF16 MFMA GEMM on activations rounded to 16 bits
// (xh; or x itself, rounded while staging: launch_gemm_float_x), and that rounding (n % 8 == 0)
hipError_t launch_mv_float(int type, bool round, const uint8_t *W, long long rb, const float *x, float *y, int N, int K,
                           int T, hipStream_t stream);
hipError_t launch_gemm_float(int type, const uint8_t *W, long long rb, const uint16_t *xh, float *y, int N, int K,
                             int T, hipStream_t stream);
hipError_t launch_gemm_float_x(int type, const uint8_t *W, long long rb, const float *x, float *y, int N, int K,
                               int T, hipStream_t stream);
hipError_t launch_round_half(int type, const float *x, uint16_t *xh, long long n, hipStream_t stream);
// fp32 activations over quantized weights (fquant.hip; with_float: F32 / F16 / BF16 too, for the expert-indexed
// forms): T dense tokens; expert-indexed (ids [T][n_used]); expert tiles of up to fq_tile() entries. s: the output
// scale, es: per-expert scales (null: s)
bool fq_type(int type, bool with_float);
int fq_tile();
hipError_t launch_fq_dense(int type, const uint8_t *W, long long rb, const float *x, float *y, int N, int K, int T,
                           float s, hipStream_t stream);
hipError_t launch_fq_id(int type, const uint8_t *W, long long rb, const int32_t *ids, int n_used, int x_per_slot,
                        const float *x, float *y, int N, int K, int T, const float *es, float s, hipStream_t stream);
hipError_t launch_fq_tiles(int type, const uint8_t *W, long long rb, const float *x, float *y, int N, int K,
                           int max_tiles, const int32_t *n_tiles, const int32_t *tile_e, const int32_t *tile_start,
                           const int32_t *tile_n, const int32_t *in_rows, const int32_t *out_rows, const float *es,
                           float s, hipStream_t stream);
// the split-Q8_0 copy of an F32 / F16 / BF16 matrix (qs [N][K], fp16 d [N][K / 32]; K % 256 == 0) and its matvec
// on a Q8_0 activation (q8, d8): lmhead.hip
hipError_t launch_quant_rows_q8_0(int type, const uint8_t *W, long long rb, int N, int K, int8_t *qs, uint16_t *d,
                                  hipStream_t stream);
hipError_t launch_mv_q8_0s(const int8_t *qs, const uint16_t *d, const int8_t *q8, const float *d8, float *y, int N,
                           int K, hipStream_t stream);
// the int8-MFMA GEMM (gemm_i8.hip: Q4_K, Q5_K, Q6_K, IQ4_XS with the Q8_K activation, xq = qK, dx = dK, xsum =
// bsK; Q8_0, MXFP4 with the Q8_0 one, xq = q0, dx = d0): dense grid (tokens / gemm_i8kq_token_tile(false), rows /
// gemm_i8kq_rows()), MoE grid (rows / gemm_i8kq_rows(), tiles) with tiles of up to gemm_i8kq_token_tile(true) entries
bool gemm_i8kq_supported(int type);
int gemm_i8kq_token_tile(bool moe);
int gemm_i8_moe_tile(int type);  // the largest expert tile of the int8 GEMMs (GemmArgs::tt: the caller's tile)
int gemm_i8kq_rows();  // weight rows per workgroup
hipError_t launch_gemm_i8kq(int type, const GemmArgs &a, dim3 grid, hipStream_t stream);

// lanes per row the decode kernels use for a matrix of K columns and `rows` rows in total
int matvec_lanes(int type, int K, long long rows);

// Decode tuning, read from the environment once per process: PURHIE_MV_TILE=0 sends every shape to the per-wave
// kernels (tile 0; qmatvec_debug_decode_path changes it at run time), PURHIE_MV_THREADS fixes the tile kernel's
// workgroup size (64 / 128 / 256, else 0 = chosen per launch), PURHIE_MV_LANES the per-wave kernels' lanes per row
// (8 .. 64, a power of two, else 0 = chosen per shape), PURHIE_MV_BALANCE=0 keeps the tile kernel's rows a tile at
// their most (balance 0) instead of fewer where that lightens the most loaded CU
struct MvTune {
    int tile, threads, lanes, balance, trim;
};
const MvTune &mv_tune();
void mv_tune_set_tile(int on);
bool mv_tile_on();  // the tile kernels on (the tuning's value, or the last mv_tune_set_tile)

}  // namespace pq
