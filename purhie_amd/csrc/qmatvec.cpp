// qmatvec.cpp -- the C ABI of include/qmatvec.h over this library's HIP kernels.
//
// Host-side dispatch keeps the reference's src/qmatvec.cpp contract (argument checks, error codes, buffer
// layout of qmatvec_q8); the launch geometry is this library's own (wave64 kernels, lanes per row chosen per
// shape, activation staged in LDS). The output-scale registry is out_scale.cpp.
#include "../../include/moe_ops.h"
#include "../../include/qmatvec.h"
#include "../../include/quant_types.h"
#include "kernels.h"
#include "out_scale.h"

#include <atomic>
#include <stdlib.h>
#include <string.h>

using namespace pq;

namespace {

bool is_int8_type(int t) {
    return t == TY_Q8_0 || t == TY_Q4_K || t == TY_Q5_K || t == TY_Q6_K || t == TY_IQ4_XS || t == TY_FP4 ||
           t == TY_FAST || t == TY_MXFP4 || t == TY_NVFP4;
}
bool reads_q8k(int t) { return t == TY_Q4_K || t == TY_Q5_K || t == TY_Q6_K || t == TY_IQ4_XS; }
int act_blk(int t) { return reads_q8k(t) ? 256 : 32; }

// required K multiple of each int8 kernel (src/qmatvec.cpp:423-429)
int k_multiple(int t) {
    switch (t) {
    case TY_Q8_0: case TY_FP4: case TY_NVFP4: return 64;
    case TY_FAST: case TY_MXFP4: return 128;
    case TY_Q4_K: case TY_Q5_K: case TY_Q6_K: case TY_IQ4_XS: return 256;
    }
    return 0;
}

// weight base alignment the kernels' loads need (Q4_K: 16-byte loads of 16-aligned blocks)
uintptr_t w_align(int t) { return t == TY_Q4_K || t == TY_Q5_K ? 16 : t == TY_IQ4_XS ? 8 : 4; }

int g_inited = 0;
std::atomic<int> g_prefill{0};
int g_prefill_fp32 = 0;

// capture mode (qmatvec_debug_capture): the integer dots of every int8 launch go to g_cap (g_cap_n ints)
int32_t *g_cap = nullptr;
size_t g_cap_n = 0;

// the capture buffer for a launch writing `need` ints, or an error when it does not fit
hipError_t cap_for(long long need, int32_t *&cap) {
    cap = g_cap;
    if (g_cap && (need < 0 || (size_t)need > g_cap_n)) return hipErrorInvalidValue;
    return hipSuccess;
}

// the output factor of a launch on rows from W (1 without a registration)
float dense_scale(const void *W) { return scale_dense(W); }

// an expert launch's factors for the stacked experts W: per-expert factors (handed to the kernel, which reads
// them on the device) or one factor for all
void expert_scale(const void *W, const float *&es, float &s) {
    es = nullptr;
    s = 1.0f;
    ScaleHit h;
    if (scale_find(W, h)) {
        if (h.n > 1) es = h.s;
        else s = h.s[0];
    }
}

void act_ptrs(int type, const qmatvec_q8 *q, const int8_t *&q8, const float *&d8, const int32_t *&bs) {
    const bool kq = reads_q8k(type);
    q8 = kq ? q->qK : q->q0;
    d8 = kq ? q->dK : q->d0;
    bs = kq ? q->bsK : nullptr;
}

// batches of at least this many tokens take the GEMM outside prefill mode (QMATVEC_WMMA_MIN_T, as the
// reference's src/qmatvec.cpp:150)
int gemm_min_t() {
    static const int v = getenv("QMATVEC_WMMA_MIN_T") ? atoi(getenv("QMATVEC_WMMA_MIN_T")) : 32;
    return v;
}

// The MFMA GEMMs are on unless QMATVEC_NO_WMMA / QMATVEC_NO_WMMA_MM is set (read once, the reference's A/B switch,
// src/qmatvec.cpp:149) or prefill-fp32 mode is on (src/qmatvec.cpp:49-52: prefill rows summed like the token by
// token decoding's). Off, batches and expert tiles run through the decode kernels, one token / entry at a time
// in the decode order.
bool mfma_on() {
    static const bool env = getenv("QMATVEC_NO_WMMA") == nullptr && getenv("QMATVEC_NO_WMMA_MM") == nullptr;
    return env && !g_prefill_fp32;
}

// expert tiles in the decode order: the tile the engine's grouping may use there (the reference's QMV_MM_TB)
constexpr int ID_DECODE_TILE = 16;

// capture mode over the split GEMM: its operands into g_cap (gemm_split_capture_layout, for the rows q holds)
void split_capture(GemmArgs &a, const qmatvec_q8 *q, int K) {
    if (!g_cap) return;
    a.cap = g_cap;
    a.cap_n = (long long)g_cap_n;
    a.cap_xr = q->max_k / K;
}

// The GEMM's arguments for the activation q, read where it is: Q8_K (qK, dK, bsK) for the K-quants, Q8_0 (q0, d0)
// for the others
GemmArgs gemm_args(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int N, int K) {
    GemmArgs a{};
    a.W = (const uint8_t *)W;
    a.row_bytes = (long long)row_bytes;
    const bool kq = reads_q8k(type);
    a.xq = kq ? q->qK : q->q0;
    a.dx = kq ? q->dK : q->d0;
    a.xsum = kq ? q->bsK : nullptr;
    a.y = y;
    a.N = N;
    a.K = K;
    return a;
}

// K multiple the GEMM of a type needs (the int8 per-block GEMM takes 64; 128 keeps the shapes it serves)
int gemm_k_mult(int type) {
    if (gemm_split(type)) return gemm_split_k_multiple();
    return type == TY_Q8_0 || type == TY_MXFP4 ? 128 : 256;
}

hipError_t gemm_dense(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, long long ldy, int N,
                      int K, int T, hipStream_t stream) {
    GemmArgs a = gemm_args(type, W, row_bytes, q, y, N, K);
    a.ldy = ldy;
    a.T = T;
    a.osc = dense_scale(W);
    if (gemm_split(type)) {
        const int BT = gemm_split_token_tile(false, T), RN = gemm_split_rows(false, T);
        a.tt = BT;
        split_capture(a, q, K);
        return launch_gemm_split(type, a, dim3((unsigned)((T + BT - 1) / BT), (unsigned)((N + RN - 1) / RN)), stream);
    }
    if (const hipError_t e = cap_for((long long)T * N * (K / gemm_cap_unit(type)), a.cap); e != hipSuccess) return e;
    const int BT = gemm_i8kq_token_tile(false), RN = gemm_i8kq_rows();
    return launch_gemm_i8kq(type, a, dim3((unsigned)((T + BT - 1) / BT), (unsigned)((N + RN - 1) / RN)), stream);
}

}  // namespace

extern "C" {

int qmatvec_init(const char *co_path) {
    (void)co_path;
    if (g_inited) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return -1;
    g_inited = 1;
    return 0;
}

void qmatvec_free(void) { g_inited = 0; }

// ---- float activations (src/qmatvec.cpp:255-366, 601-671): F32 / F16 / BF16 weights through fmat.hip (decode
// matvec, MFMA GEMM), the quantized types (Q8_0, K-quants, IQ4_XS, the FP4 family) through fquant.hip's kernel (fp32
// activations against the exactly decoded weights), expert-indexed forms of both through fquant.hip. Other types
// return hipErrorInvalidDeviceFunction, the reference's answer for a missing kernel.
namespace {
bool float_type(int t) { return t == QT_F32 || t == QT_F16 || t == QT_BF16; }
bool half_type(int t) { return t == QT_F16 || t == QT_BF16; }
bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// the reference's shape checks: K a whole number of blocks, row_bytes the type's row size
bool float_shape_ok(int type, size_t row_bytes, int K) {
    const qt_traits *tr = qt_get_traits(type);
    return tr && K > 0 && K % tr->blck_size == 0 && row_bytes == qt_row_size(type, K);
}

// the decode kernel over T tokens, after the reference's argument checks
hipError_t float_rows(int type, bool round, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                      int T, hipStream_t stream) {
    if (!float_type(type) && !fq_type(type, false)) return hipErrorInvalidDeviceFunction;
    if (!W || !x || !y || N < 0 || T < 1 || !float_shape_ok(type, row_bytes, K)) return hipErrorInvalidValue;
    if (N == 0) return hipSuccess;
    if (!float_type(type))
        return launch_fq_dense(type, (const uint8_t *)W, (long long)row_bytes, x, y, N, K, T, dense_scale(W), stream);
    return launch_mv_float(type, round, (const uint8_t *)W, (long long)row_bytes, x, y, N, K, T, stream);
}
}  // namespace

int qmatvec_supported(int type) { return float_type(type) || fq_type(type, false) ? 1 : 0; }

hipError_t qmatvec_launch_bf16f(const void *W, size_t row_bytes, const float *x, float *y, int N, int K, int T,
                                hipStream_t stream) {
    if (!W || !x || !y || T < 1 || row_bytes != (size_t)K * 2) return hipErrorInvalidValue;
    return float_rows(QT_BF16, false, W, row_bytes, x, y, N, K, T, stream);
}

hipError_t qmatvec_launch(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                          hipStream_t stream) {
    return float_rows(type, true, W, row_bytes, x, y, N, K, 1, stream);
}

int qmatvec_half_supported(int type, const void *W, size_t row_bytes, int N, int K, int T) {
    return half_type(type) && mfma_on() && (g_prefill || T >= gemm_min_t()) && T >= 1 && N >= 64 && K > 0 &&
           K % 8 == 0 && K < (1 << 22) && row_bytes >= (size_t)K * 2 && row_bytes % 16 == 0 &&
           row_bytes < ((size_t)1 << 23) && al16(W);
}

hipError_t qmatvec_round_half(int type, const float *x, uint16_t *xh, long long n, hipStream_t stream) {
    if (!half_type(type)) return hipErrorInvalidDeviceFunction;
    if (!x || !xh || n < 0 || n % 8 != 0 || !al16(x) || !al16(xh)) return hipErrorInvalidValue;
    return launch_round_half(type, x, xh, n, stream);
}

hipError_t qmatvec_launch_batch_hx(int type, const void *W, size_t row_bytes, const uint16_t *xh, float *y, int N,
                                   int K, int T, hipStream_t stream) {
    if (!qmatvec_half_supported(type, W, row_bytes, N, K, T)) return hipErrorInvalidDeviceFunction;
    if (!xh || !y || !al16(xh)) return hipErrorInvalidValue;
    return launch_gemm_float(type, (const uint8_t *)W, (long long)row_bytes, xh, y, N, K, T, stream);
}

hipError_t qmatvec_launch_batch(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                                int T, hipStream_t stream) {
    return qmatvec_launch_batch_h(type, W, row_bytes, x, nullptr, 0, y, N, K, T, stream);
}

// F16 / BF16 batches the GEMM takes: x rounded to 16 bits first into the caller's scratch buffer xh when it holds
// T K values (the GEMM then reads 16-bit activations: half the bytes of rounding fp32 ones while staging, measured
// 2x faster), else the GEMM reading x and rounding it while staging (the reference's matmul_wmma_f, src/qmatvec.cpp:
// 341-352); every other batch through the decode kernel, token by token in its order. Nothing is allocated.
hipError_t qmatvec_launch_batch_h(int type, const void *W, size_t row_bytes, const float *x, uint16_t *xh,
                                  size_t xh_bytes, float *y, int N, int K, int T, hipStream_t stream) {
    if (qmatvec_half_supported(type, W, row_bytes, N, K, T) && x && y && al16(x) && (!xh || al16(xh))) {
        if (xh && xh_bytes >= (size_t)T * K * 2) {
            const hipError_t e = qmatvec_round_half(type, x, xh, (long long)T * K, stream);
            return e != hipSuccess ? e : qmatvec_launch_batch_hx(type, W, row_bytes, xh, y, N, K, T, stream);
        }
        return launch_gemm_float_x(type, (const uint8_t *)W, (long long)row_bytes, x, y, N, K, T, stream);
    }
    return float_rows(type, true, W, row_bytes, x, y, N, K, T, stream);
}
// The split-Q8_0 copy of a float matrix (the opt-in LM head, src/qmatvec.cpp:369-390): ggml's Q8_0 quantization
// per 32 values into qs [N][K] (16-byte aligned) and fp16 d [N][K / 32]; y = qs x on the activation's Q8_0 part
int qmatvec_q8_0s_source_supported(int type, int K) { return K > 0 && K % 256 == 0 && float_type(type) ? 1 : 0; }

hipError_t qmatvec_quantize_rows_q8_0(int type, const void *W, size_t row_bytes, int N, int K, int8_t *qs, uint16_t *d,
                                      hipStream_t stream) {
    if (!qmatvec_q8_0s_source_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (row_bytes != qt_row_size(type, K) || !al16(qs) || !W || !d || N < 0) return hipErrorInvalidValue;
    return launch_quant_rows_q8_0(type, (const uint8_t *)W, (long long)row_bytes, N, K, qs, d, stream);
}

hipError_t qmatvec_launch_q8_0s(const int8_t *qs, const uint16_t *d, const qmatvec_q8 *q, float *y, int N, int K,
                                hipStream_t stream) {
    if (!q || K <= 0 || K % 256 != 0 || K > q->max_k || !al16(qs) || !d || !y || !q->q0 || !q->d0 || N < 0)
        return hipErrorInvalidValue;
    return launch_mv_q8_0s(qs, d, q->q0, q->d0, y, N, K, stream);
}
// One token of the low-rank up projection (src/qmatvec.cpp:467-479): y = W x, x = SiLU(lo scale) zero-padded from
// n to K values and quantized to Q8_0 inside the kernel, the bits that SwiGLU(lo scale, 1)'s quantization followed by
// qmatvec_launch_q8 give (no output scale, as the reference's kernel). ROCmFP4_FAST, K % 128 == 0, K <= 1024.
int qmatvec_q8_lr_supported(int type, int K) {
    return type == QT_Q4_0_ROCMFP4_FAST && K > 0 && K % 128 == 0 && K <= LR_MAXK ? 1 : 0;
}

hipError_t qmatvec_launch_q8_lr(int type, const void *W, size_t row_bytes, const float *lo, int n, int K, float scale,
                                float *y, int N, hipStream_t stream) {
    if (!qmatvec_q8_lr_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (n < 0 || n > K || row_bytes != qt_row_size(type, K) || row_bytes % 4 != 0 || ((uintptr_t)W & 3) != 0 || !W ||
        !y || (n > 0 && !lo) || N < 0)
        return hipErrorInvalidValue;
    if (N == 0) return hipSuccess;
    MvArgs a{};
    for (int i = 0; i < 4; ++i) {
        a.W[i] = (const uint8_t *)W;
        a.y[i] = y;
        a.bound[i] = N;
        a.ystride[i] = N;
        a.osc[i] = 1.0f;
    }
    a.row_bytes = (long long)row_bytes;
    a.Nt = N;
    a.K = K;
    a.T = 1;
    a.L = matvec_lanes(type, K, N);
    a.lr_lo = lo ? lo : y;  // (n == 0: never read)
    a.lr_n = n;
    a.lr_scale = scale;
    return launch_matvec_lr(type, a, stream);
}
// Float expert-indexed matvecs: for token t and slot j, expert e = ids[t n_used + j] (rows e N .. e N + N - 1 of W)
// times input row t (x_per_slot 0) or t n_used + j into output row t n_used + j; an id below 0 writes nothing.
hipError_t qmatvec_launch_id(int type, const void *W, size_t row_bytes, const int32_t *ids, int n_used, int x_per_slot,
                             const float *x, float *y, int N, int K, int T, hipStream_t stream) {
    if (!fq_type(type, true)) return hipErrorInvalidDeviceFunction;
    if (T <= 0 || n_used <= 0 || !float_shape_ok(type, row_bytes, K)) return hipErrorInvalidValue;
    if (!W || !ids || !x || !y || N < 0) return hipErrorInvalidValue;
    if (N == 0) return hipSuccess;
    const float *es;
    float s;
    expert_scale(W, es, s);
    return launch_fq_id(type, (const uint8_t *)W, (long long)row_bytes, ids, n_used, x_per_slot, x, y, N, K, T, es, s,
                        stream);
}

int qmatvec_id_batch_f_supported(int type) { return fq_type(type, true) ? 1 : 0; }

// The same over expert tiles (the grouping's tiles of up to `tile` <= 16 entries): each entry gets the bits
// qmatvec_launch_id gives it
hipError_t qmatvec_launch_id_batch_f(int type, const void *W, size_t row_bytes, const float *x, float *y, int N, int K,
                                     int max_tiles, int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                     const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                     const int32_t *out_rows, hipStream_t stream) {
    if (!qmatvec_id_batch_f_supported(type)) return hipErrorInvalidDeviceFunction;
    if (max_tiles <= 0 || tile <= 0 || tile > fq_tile() || !float_shape_ok(type, row_bytes, K))
        return hipErrorInvalidValue;
    if (!W || !x || !y || !n_tiles || !tile_e || !tile_start || !tile_n || !in_rows || !out_rows || N < 0)
        return hipErrorInvalidValue;
    if (N == 0) return hipSuccess;
    const float *es;
    float s;
    expert_scale(W, es, s);
    return launch_fq_tiles(type, (const uint8_t *)W, (long long)row_bytes, x, y, N, K, max_tiles, n_tiles, tile_e,
                           tile_start, tile_n, in_rows, out_rows, es, s, stream);
}

void qmatvec_set_prefill(int on) { g_prefill = on && !getenv("QMATVEC_PREFILL_SPLIT_VARIANT"); }
int qmatvec_prefill(void) { return g_prefill; }
void qmatvec_set_prefill_fp32(int on) { g_prefill_fp32 = on; }

static size_t align16(size_t n) { return (n + 15) & ~(size_t)15; }

size_t qmatvec_q8_bytes(int max_k) {
    const size_t k = (size_t)max_k;
    return 2 * align16(k) + 2 * align16(k / 32 * 4) + align16(k / 256 * 4) + align16(k / 16 * 4);
}

void qmatvec_q8_bind(qmatvec_q8 *q, void *mem, int max_k) {
    const size_t k = (size_t)max_k;
    char *p = (char *)mem;
    q->q0 = (int8_t *)p;
    p += align16(k);
    q->qK = (int8_t *)p;
    p += align16(k);
    q->d0 = (float *)p;
    p += align16(k / 32 * 4);
    q->dK = (float *)p;
    p += align16(k / 256 * 4);
    q->bsK = (int32_t *)p;
    p += align16(k / 16 * 4);
    q->s0 = (int32_t *)p;
    q->max_k = max_k;
    q->xh = nullptr;
    q->xh_bf16 = 0;
}

int qmatvec_q8_supported(int type, int K) {
    if (!is_int8_type(type) || K <= 0) return 0;
    return K % k_multiple(type) == 0;
}

hipError_t qmatvec_quantize(const float *x, int K, const qmatvec_q8 *q, hipStream_t stream) {
    if (!q || !x) return hipErrorInvalidValue;
    if (K <= 0 || K % 32 != 0 || K > q->max_k) return hipErrorInvalidValue;
    Q8Ptrs o{q->q0, q->d0, q->qK, q->dK, q->bsK, q->s0};
    return launch_quantize_q8(x, K, o, stream);
}

int qmatvec_q8_few_supported(int type, int K, int T) { return T >= 1 && T <= 4 && qmatvec_q8_supported(type, K); }

hipError_t qmatvec_launch_q8_multi_t(int type, int n, const void *const *Ws, const int *Ns, float *const *ys,
                                     size_t row_bytes, const qmatvec_q8 *q, int K, int T, hipStream_t stream) {
    if (!qmatvec_q8_few_supported(type, K, T)) return hipErrorInvalidDeviceFunction;
    if (!q || n < 1 || n > 4 || row_bytes != qt_row_size(type, K) || (long long)K * T > q->max_k)
        return hipErrorInvalidValue;
    MvArgs a{};
    int Nt = 0;
    for (int i = 0; i < 4; ++i) {
        const int j = i < n ? i : n - 1;  // unused slots repeat the last matrix, with no rows
        if (((uintptr_t)Ws[j] & (w_align(type) - 1)) != 0 || Ns[j] < 0) return hipErrorInvalidValue;
        a.W[i] = (const uint8_t *)Ws[j];
        a.y[i] = ys[j];
        if (i < n) Nt += Ns[i];
        a.bound[i] = Nt;
        a.ystride[i] = Ns[j];
        a.osc[i] = dense_scale(Ws[j]);
    }
    if (Nt == 0) return hipSuccess;
    a.row_bytes = (long long)row_bytes;
    act_ptrs(type, q, a.q, a.d, a.bs);
    a.Nt = Nt;
    a.K = K;
    a.T = T;
    a.L = matvec_lanes(type, K, Nt);
    if (const hipError_t e = cap_for((long long)T * Nt * (K / cap_group(type)), a.cap); e != hipSuccess) return e;
    return launch_matvec(type, a, stream);
}

hipError_t qmatvec_launch_q8_multi(int type, int n, const void *const *Ws, const int *Ns, float *const *ys,
                                   size_t row_bytes, const qmatvec_q8 *q, int K, hipStream_t stream) {
    return qmatvec_launch_q8_multi_t(type, n, Ws, Ns, ys, row_bytes, q, K, 1, stream);
}

hipError_t qmatvec_launch_q8_pair(int type, const void *W, int N, float *y, const void *W2, int N2, float *y2,
                                  size_t row_bytes, const qmatvec_q8 *q, int K, hipStream_t stream) {
    const void *Ws[] = {W, W2};
    const int Ns[] = {N, N2};
    float *ys[] = {y, y2};
    return qmatvec_launch_q8_multi(type, 2, Ws, Ns, ys, row_bytes, q, K, stream);
}

hipError_t qmatvec_launch_q8(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int N, int K,
                             hipStream_t stream) {
    const void *Ws[] = {W};
    const int Ns[] = {N};
    float *ys[] = {y};
    return qmatvec_launch_q8_multi(type, 1, Ws, Ns, ys, row_bytes, q, K, stream);
}

hipError_t qmatvec_launch_q8_id_x(int type, const void *W, const void *W2, const void *Wx, const void *W2x,
                                  size_t row_bytes, const int32_t *ids, int n_used, int x_per_slot,
                                  const qmatvec_q8 *q, float *y, float *y2, int N, int K, int T, hipStream_t stream) {
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (!q) return hipErrorInvalidValue;
    const long long in_rows = (long long)T * (x_per_slot ? n_used : 1);
    const uintptr_t am = w_align(type) - 1;
    if (T <= 0 || n_used <= 0 || N <= 0 || row_bytes != qt_row_size(type, K) || ((uintptr_t)W & am) != 0 ||
        in_rows * K > q->max_k)
        return hipErrorInvalidValue;
    if ((((uintptr_t)W2 | (uintptr_t)Wx | (uintptr_t)W2x) & am) != 0) return hipErrorInvalidValue;
    MvIdArgs a{};
    a.W[0] = (const uint8_t *)W;
    a.W[1] = (const uint8_t *)W2;
    a.Wx[0] = (const uint8_t *)Wx;
    a.Wx[1] = (const uint8_t *)W2x;
    a.y[0] = y;
    a.y[1] = y2;
    const void *ws[2] = {W, W2}, *wx[2] = {Wx, W2x};
    for (int m = 0; m < 2; ++m) {
        expert_scale(ws[m], a.es[m], a.s[m]);  // (per-expert factors are read by the kernel: device-visible)
        a.sx[m] = wx[m] ? dense_scale(wx[m]) : 1.0f;
    }
    a.row_bytes = (long long)row_bytes;
    a.ids = ids;
    act_ptrs(type, q, a.q, a.d, a.bs);
    a.n_used = n_used;
    a.x_per_slot = x_per_slot;
    a.N = N;
    a.K = K;
    a.T = T;
    a.nmat = W2 ? 2 : 1;
    a.L = matvec_lanes(type, K, (long long)N * n_used * a.nmat * T);
    a.cap_rows = (long long)T * n_used;
    if (const hipError_t e = cap_for(a.nmat * a.cap_rows * N * (K / cap_group(type)), a.cap); e != hipSuccess) return e;
    return launch_matvec_id(type, a, stream);
}

hipError_t qmatvec_launch_q8_id_pair_routed(int type, const void *W, const void *W2, size_t row_bytes,
                                            const float *logits, int n_expert, int32_t *ids, float *wts, int n_used,
                                            const qmatvec_q8 *q, float *y, float *y2, int N, int K, int T,
                                            hipStream_t stream) {
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    const uintptr_t am = w_align(type) - 1;
    if (!logits || !ids || !wts || !W || !W2 || !q || !y || !y2 || T <= 0 || n_used <= 0 || n_expert < n_used ||
        N <= 0 || row_bytes != qt_row_size(type, K) || (((uintptr_t)W | (uintptr_t)W2) & am) != 0 ||
        (long long)T * K > q->max_k)
        return hipErrorInvalidValue;
    auto two_launches = [&]() {
        const hipError_t e = gpu_moe_router(logits, nullptr, nullptr, ids, wts, nullptr, n_expert, n_used, 0, T,
                                            stream, 0);
        return e != hipSuccess ? e : qmatvec_launch_q8_id_pair(type, W, W2, row_bytes, ids, n_used, 0, q, y, y2, N,
                                                               K, T, stream);
    };
    if (n_expert > 256 || n_used > 64 || !mv_tile_on()) return two_launches();
    MvIdArgs a{};
    a.W[0] = (const uint8_t *)W;
    a.W[1] = (const uint8_t *)W2;
    a.y[0] = y;
    a.y[1] = y2;
    const void *ws[2] = {W, W2};
    for (int m = 0; m < 2; ++m) {
        expert_scale(ws[m], a.es[m], a.s[m]);
        a.sx[m] = 1.0f;
    }
    a.row_bytes = (long long)row_bytes;
    act_ptrs(type, q, a.q, a.d, a.bs);
    a.n_used = n_used;
    a.x_per_slot = 0;
    a.N = N;
    a.K = K;
    a.T = T;
    a.nmat = 2;
    a.L = matvec_lanes(type, K, (long long)N * n_used * 2 * T);
    a.route_logits = logits;
    a.route_ne = n_expert;
    a.route_ids = ids;
    a.route_wts = wts;
    const hipError_t e = launch_matvec_id_tile(type, a, stream);
    return e == hipErrorNotSupported ? two_launches() : e;
}

int qmatvec_q8_id_swiglu_supported(int type, int K) {
    return qmatvec_q8_supported(type, K) && matvec_id_swiglu_supported(type, K) ? 1 : 0;
}

// the expert down matvec of a decode step with the SwiGLU launch folded in: entry (t, slot) reads row
// t * n_used + slot of g and u, and the kernel quantizes SwiGLU of it to Q8_0 as gpu_swiglu's fused quantizer
// would, so y is bit-identical to gpu_swiglu(g, u, .., q8) followed by qmatvec_launch_q8_id(.., x_per_slot = 1, q8)
hipError_t qmatvec_launch_q8_id_swiglu(int type, const void *W, const void *Wx, size_t row_bytes, const int32_t *ids,
                                       int n_used, const float *g, const float *u, float *y, int N, int K, int T,
                                       hipStream_t stream) {
    if (!qmatvec_q8_id_swiglu_supported(type, K)) return hipErrorInvalidDeviceFunction;
    const uintptr_t am = w_align(type) - 1;
    if (!W || !ids || !g || !u || !y || T <= 0 || n_used <= 0 || N <= 0 || row_bytes != qt_row_size(type, K) ||
        ((uintptr_t)W & am) != 0 || ((uintptr_t)Wx & am) != 0)
        return hipErrorInvalidValue;
    MvIdArgs a{};
    a.W[0] = (const uint8_t *)W;
    a.Wx[0] = (const uint8_t *)Wx;
    a.y[0] = y;
    a.es[1] = nullptr;
    a.s[1] = a.sx[1] = 1.0f;
    expert_scale(W, a.es[0], a.s[0]);
    a.sx[0] = Wx ? dense_scale(Wx) : 1.0f;
    a.row_bytes = (long long)row_bytes;
    a.ids = ids;
    a.sw_g = g;
    a.sw_u = u;
    a.n_used = n_used;
    a.x_per_slot = 1;
    a.N = N;
    a.K = K;
    a.T = T;
    a.nmat = 1;
    a.L = matvec_lanes(type, K, (long long)N * n_used * T);
    a.cap_rows = (long long)T * n_used;
    if (const hipError_t e = cap_for(a.cap_rows * N * (K / cap_group(type)), a.cap); e != hipSuccess) return e;
    return launch_matvec_id(type, a, stream);
}

hipError_t qmatvec_launch_q8_id(int type, const void *W, size_t row_bytes, const int32_t *ids, int n_used,
                                int x_per_slot, const qmatvec_q8 *q, float *y, int N, int K, int T, hipStream_t stream) {
    return qmatvec_launch_q8_id_x(type, W, nullptr, nullptr, nullptr, row_bytes, ids, n_used, x_per_slot, q, y,
                                  nullptr, N, K, T, stream);
}

hipError_t qmatvec_launch_q8_id_pair(int type, const void *W, const void *W2, size_t row_bytes, const int32_t *ids,
                                     int n_used, int x_per_slot, const qmatvec_q8 *q, float *y, float *y2, int N, int K,
                                     int T, hipStream_t stream) {
    return qmatvec_launch_q8_id_x(type, W, W2, nullptr, nullptr, row_bytes, ids, n_used, x_per_slot, q, y, y2, N, K,
                                  T, stream);
}

hipError_t qmatvec_launch_q8_batch(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y,
                                   long long ldy, int N, int K, int T, hipStream_t stream) {
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (!q || T <= 0 || N <= 0 || row_bytes != qt_row_size(type, K) || ((uintptr_t)W & (w_align(type) - 1)) != 0 ||
        (long long)T * K > q->max_k || ldy < N)
        return hipErrorInvalidValue;
    // prefill mode or a batch of 32+ tokens: the MFMA GEMM (the reference's WMMA threshold, src/qmatvec.cpp:553)
    if (mfma_on() && gemm_supported(type) && K % gemm_k_mult(type) == 0 && (g_prefill || T >= gemm_min_t()) &&
        N >= 64)
        return gemm_dense(type, W, row_bytes, q, y, ldy, N, K, T, stream);
    // tokens in groups of up to 4 through the decode kernel (weights read once per group)
    MvArgs a{};
    a.W[0] = a.W[1] = a.W[2] = a.W[3] = (const uint8_t *)W;
    a.bound[0] = a.bound[1] = a.bound[2] = a.bound[3] = N;
    a.ystride[0] = a.ystride[1] = a.ystride[2] = a.ystride[3] = ldy;
    a.osc[0] = a.osc[1] = a.osc[2] = a.osc[3] = dense_scale(W);
    a.row_bytes = (long long)row_bytes;
    a.Nt = N;
    a.K = K;
    a.L = matvec_lanes(type, K, N);
    const int8_t *q8;
    const float *d8;
    const int32_t *bs;
    act_ptrs(type, q, q8, d8, bs);
    const int kb = K / act_blk(type);
    int32_t *cap;
    if (const hipError_t e = cap_for((long long)T * N * (K / cap_group(type)), cap); e != hipSuccess) return e;
    for (int t0 = 0; t0 < T; t0 += 4) {
        a.cap = cap ? cap + (long long)t0 * N * (K / cap_group(type)) : nullptr;
        a.T = T - t0 < 4 ? T - t0 : 4;
        a.y[0] = a.y[1] = a.y[2] = a.y[3] = y + (long long)t0 * ldy;
        a.q = q8 + (long long)t0 * K;
        a.d = d8 + (long long)t0 * kb;
        a.bs = bs ? bs + (long long)t0 * (K / 16) : nullptr;
        const hipError_t e = launch_matvec(type, a, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int qmatvec_q8_id_batch_supported(int type, int K) { return qmatvec_q8_supported(type, K); }

static bool id_gemm_ok(int type, int N, int K) {
    return mfma_on() && gemm_supported(type) && K % gemm_k_mult(type) == 0 && N >= 64;
}

// the largest tile the expert-tiled launch takes: the GEMM reads each expert's weights once per this many
// entries; the decode-order path takes the reference's 16 (src/qmatvec.cpp:612-615)
int qmatvec_id_batch_tile(int type, int N, int K) {
    if (!id_gemm_ok(type, N, K)) return ID_DECODE_TILE;
    return gemm_split(type) ? gemm_split_token_tile(true, 0) : gemm_i8_moe_tile(type);
}

// the expert-tiled GEMM over W (and W2, the pair's second matrix, or null), the activation read in place: input
// rows are in_rows[] of q
static hipError_t id_gemm(int type, const void *W, const void *W2, size_t row_bytes, const qmatvec_q8 *q, float *y,
                          float *y2, int N, int K, int max_tiles, int tile, const int32_t *n_tiles,
                          const int32_t *tile_e, const int32_t *tile_start, const int32_t *tile_n,
                          const int32_t *in_rows, const int32_t *out_rows, hipStream_t stream) {
    GemmArgs a = gemm_args(type, W, row_bytes, q, y, N, K);
    a.tt = tile;
    a.n_tiles = n_tiles;
    a.tile_e = tile_e;
    a.tile_start = tile_start;
    a.tile_n = tile_n;
    a.in_rows = in_rows;
    a.out_rows = out_rows;
    expert_scale(W, a.es, a.osc);
    const bool split = gemm_split(type);
    const int RN = split ? gemm_split_rows(true, 0) : gemm_i8kq_rows(), rt = (N + RN - 1) / RN;
    if (W2) {
        a.W2 = (const uint8_t *)W2;
        a.y2 = y2;
        expert_scale(W2, a.es2, a.osc2);
        a.rt = rt;
    }
    const dim3 grid((unsigned)(W2 ? 2 * rt : rt), (unsigned)max_tiles);
    if (split) {
        if (!W2) split_capture(a, q, K);
        return launch_gemm_split(type, a, grid, stream);
    }
    a.cap = W2 ? nullptr : g_cap;  // (tiles mode: rows from out_rows; the caller sizes the buffer)
    return launch_gemm_i8kq(type, a, grid, stream);
}

hipError_t qmatvec_launch_q8_id_batch(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int N,
                                      int K, int max_tiles, int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                      const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                      const int32_t *out_rows, hipStream_t stream) {
    if (!qmatvec_q8_id_batch_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (!q || max_tiles <= 0 || tile <= 0 || tile > qmatvec_id_batch_tile(type, N, K) || N <= 0 ||
        row_bytes != qt_row_size(type, K) || ((uintptr_t)W & (w_align(type) - 1)) != 0)
        return hipErrorInvalidValue;
    if (!id_gemm_ok(type, N, K)) {  // the decode kernels, one entry per block
        MvIdArgs a{};
        a.W[0] = (const uint8_t *)W;
        a.y[0] = y;
        a.sx[0] = 1.0f;
        expert_scale(W, a.es[0], a.s[0]);
        a.row_bytes = (long long)row_bytes;
        act_ptrs(type, q, a.q, a.d, a.bs);
        a.N = N;
        a.K = K;
        a.T = 1;
        a.n_used = 1;
        a.nmat = 1;
        a.n_tiles = n_tiles;
        a.tile_e = tile_e;
        a.tile_start = tile_start;
        a.tile_n = tile_n;
        a.in_rows = in_rows;
        a.out_rows = out_rows;
        a.tile = tile;
        a.max_tiles = max_tiles;
        a.L = matvec_lanes(type, K, (long long)N * tile * max_tiles);
        a.cap = g_cap;  // (tiles mode: output rows come from out_rows on the device; the caller sizes the buffer)
        a.cap_rows = 0;
        return launch_matvec_id(type, a, stream);
    }
    return id_gemm(type, W, nullptr, row_bytes, q, y, nullptr, N, K, max_tiles, tile, n_tiles, tile_e, tile_start,
                   tile_n, in_rows, out_rows, stream);
}

// the gate and up projections of the experts over the same tiles in one expert-tiled GEMM launch (no counterpart in
// the reference, whose engine runs qmatvec_launch_q8_id_batch twice): the same outputs bit for bit
hipError_t qmatvec_launch_q8_id_batch_pair(int type, const void *W, const void *W2, size_t row_bytes,
                                           const qmatvec_q8 *q, float *y, float *y2, int N, int K, int max_tiles,
                                           int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                           const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                           const int32_t *out_rows, hipStream_t stream) {
    if (!qmatvec_q8_id_batch_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (!q || !W2 || !y2 || max_tiles <= 0 || tile <= 0 || tile > qmatvec_id_batch_tile(type, N, K) || N <= 0 ||
        row_bytes != qt_row_size(type, K) || (((uintptr_t)W | (uintptr_t)W2) & (w_align(type) - 1)) != 0)
        return hipErrorInvalidValue;
    if (!id_gemm_ok(type, N, K) || g_cap) {  // the decode-order kernels, or a capture: two launches
        const hipError_t e = qmatvec_launch_q8_id_batch(type, W, row_bytes, q, y, N, K, max_tiles, tile, n_tiles,
                                                        tile_e, tile_start, tile_n, in_rows, out_rows, stream);
        return e != hipSuccess ? e
                               : qmatvec_launch_q8_id_batch(type, W2, row_bytes, q, y2, N, K, max_tiles, tile, n_tiles,
                                                            tile_e, tile_start, tile_n, in_rows, out_rows, stream);
    }
    return id_gemm(type, W, W2, row_bytes, q, y, y2, N, K, max_tiles, tile, n_tiles, tile_e, tile_start, tile_n, in_rows,
                   out_rows, stream);
}

// the pair with SwiGLU and its Q8_0 quantization in the epilogue (no counterpart in the reference: its engine runs
// the two GEMMs, then gpu_swiglu): h's rows out_rows[] get the bits gpu_swiglu's quantizer would write (q0, d0, and
// s0 where h binds it; the Q8_K side is not written)
int qmatvec_q8_id_batch_swiglu_supported(int type, int N, int K) {
    return qmatvec_q8_id_batch_supported(type, K) && id_gemm_ok(type, N, K) && gemm_split(type) &&
                   N % gemm_split_swiglu_rows() == 0
               ? 1
               : 0;
}

hipError_t qmatvec_launch_q8_id_batch_swiglu(int type, const void *W, const void *W2, size_t row_bytes,
                                             const qmatvec_q8 *q, const qmatvec_q8 *h, int N, int K, int max_tiles,
                                             int tile, const int32_t *n_tiles, const int32_t *tile_e,
                                             const int32_t *tile_start, const int32_t *tile_n, const int32_t *in_rows,
                                             const int32_t *out_rows, hipStream_t stream) {
    if (!qmatvec_q8_id_batch_swiglu_supported(type, N, K)) return hipErrorInvalidDeviceFunction;
    if (!q || !h || !h->q0 || !h->d0 || !W || !W2 || max_tiles <= 0 || tile <= 0 ||
        tile > qmatvec_id_batch_tile(type, N, K) || row_bytes != qt_row_size(type, K) ||
        (((uintptr_t)W | (uintptr_t)W2) & (w_align(type) - 1)) != 0)
        return hipErrorInvalidValue;
    GemmArgs a = gemm_args(type, W, row_bytes, q, nullptr, N, K);
    a.n_tiles = n_tiles;
    a.tile_e = tile_e;
    a.tile_start = tile_start;
    a.tile_n = tile_n;
    a.in_rows = in_rows;
    a.out_rows = out_rows;
    expert_scale(W, a.es, a.osc);
    a.W2 = (const uint8_t *)W2;
    expert_scale(W2, a.es2, a.osc2);
    a.hq = h->q0;
    a.hd = h->d0;
    a.hs = h->s0;
    return launch_gemm_split(type, a, dim3((unsigned)(N / gemm_split_swiglu_rows()), (unsigned)max_tiles), stream);
}

hipError_t qmatvec_debug_gemm_f8f6f4(const void *W, size_t row_bytes, const qmatvec_q8 *q, float *y, int ldy, int N,
                                     int K, int T, hipStream_t stream) {
    if (!W || !q || !y || N <= 0 || T <= 0 || K <= 0 || K % 64 != 0 || ldy < N ||
        row_bytes != qt_row_size(TY_FP4, K) || ((uintptr_t)W & 3) != 0 || (long long)T * K > q->max_k)
        return hipErrorInvalidValue;
    GemmArgs a = gemm_args(TY_FP4, W, row_bytes, q, y, N, K);
    a.ldy = ldy;
    a.T = T;
    a.osc = dense_scale(W);
    return launch_gemm_f8_exact(a, stream);
}

hipError_t qmatvec_debug_capture(int32_t *out, size_t n_ints) {
    g_cap = out;
    g_cap_n = out ? n_ints : 0;
    return hipSuccess;
}

int qmatvec_debug_capture_unit(int type, int gemm) {
    if (!is_int8_type(type)) return 0;
    return gemm ? gemm_cap_unit(type) : cap_group(type);
}

int qmatvec_debug_decode_path(int mode) {
    const int prev = mv_tune().tile;
    if (mode == 0 || mode == 1) mv_tune_set_tile(mode);
    return prev;
}

hipError_t qmatvec_debug_block_dots(int type, const void *W, size_t row_bytes, const qmatvec_q8 *q, int32_t *out,
                                    int N, int K, hipStream_t stream) {
    if (!qmatvec_q8_supported(type, K)) return hipErrorInvalidDeviceFunction;
    if (!q || !out || N <= 0 || row_bytes != qt_row_size(type, K) || K > q->max_k) return hipErrorInvalidValue;
    return launch_block_dots(type, (const uint8_t *)W, (long long)row_bytes, reads_q8k(type) ? q->qK : q->q0, out, N, K,
                             stream);
}

}  // extern "C"
