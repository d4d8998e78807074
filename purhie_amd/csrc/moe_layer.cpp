// moe_layer.cpp -- one MoE FFN as one library call (include/moe_layer.h): the engine's moe_core /
// moe_core_one / shared_as_slot (reference src/qwen_model.cpp:1093-1166) over this library's launches. Host
// code only: it lays out the caller's workspace and issues the launches on the caller's stream.
#include "../../include/moe_layer.h"
#include "../../include/moe_ops.h"
#include "../../include/qmatvec.h"
#include "../../include/quant_types.h"

#include <algorithm>
#include <cmath>
#include <mutex>

// purhie_moe_ffn_noalloc's workspace: one static device array on each GPU the library runs on (the runtime places it
// when it loads the code object on that device; it stays until the process ends)
static __device__ __align__(256) unsigned char scratch[PURHIE_MOE_SCRATCH_BYTES];

namespace {

constexpr int GROUP_MIN_T = 8;  // batches from this size group their entries by expert (src/qwen_model.cpp:1142)

bool float_router(int t) { return t == QT_F32 || t == QT_F16 || t == QT_BF16; }

bool has_shexp(const purhie_moe_weights *w) { return w->gate_shexp && w->up_shexp && w->down_shexp; }

// src/qwen_model.cpp:1095-1103: the shared expert has the routed experts' width, types and row sizes
bool slot_form(const purhie_moe_weights *w) {
    return has_shexp(w) && w->n_ff_shexp == w->n_ff_exp && w->type_shexp_gate_up == w->type_gate_up &&
           w->type_shexp_down == w->type_down && w->rb_shexp_gate_up == w->rb_gate_up &&
           w->rb_shexp_down == w->rb_down;
}

long long round256(long long n) { return (n + 255) / 256 * 256; }

// the workspace regions, each 256-byte aligned
struct Layout {
    float *logits = nullptr, *wts = nullptr, *sg = nullptr, *g = nullptr, *u = nullptr;
    float *down = nullptr, *ffg = nullptr, *ffu = nullptr, *sact = nullptr, *shout = nullptr;
    int32_t *ids = nullptr, *tok = nullptr, *pair = nullptr, *ntiles = nullptr, *te = nullptr, *ts = nullptr,
            *tn = nullptr;
    void *qx = nullptr, *qs = nullptr;
    uint16_t *xh = nullptr;  // a 16-bit copy of xn for an F16 / BF16 router's GEMM
    int ns = 0, tile = 0, max_tiles = 0, qx_k = 0, qs_k = 0;
    bool slot = false, grouped = false;
    size_t bytes = 0;
};

bool valid(const purhie_moe_weights *w, int T) {
    if (!w || T < 1 || w->n_embd <= 0 || w->n_ff_exp <= 0 || w->n_expert <= 0 || w->n_expert > 1024 ||
        w->n_expert_used < 1 || w->n_expert_used > 63 || w->n_expert_used > w->n_expert)
        return false;
    if (!w->gate_exps || !w->up_exps || !w->down_exps || !w->router) return false;
    const int E = w->n_embd, FE = w->n_ff_exp;
    if (!qmatvec_q8_supported(w->type_gate_up, E) || !qmatvec_q8_supported(w->type_down, FE)) return false;
    if (w->rb_gate_up != qt_row_size(w->type_gate_up, E) || w->rb_down != qt_row_size(w->type_down, FE)) return false;
    if (w->rb_router != qt_row_size(w->type_router, E)) return false;
    if (!qmatvec_q8_supported(w->type_router, E) && !float_router(w->type_router)) return false;
    if (has_shexp(w)) {
        const int FS = w->n_ff_shexp;
        if (FS <= 0 || !qmatvec_q8_supported(w->type_shexp_gate_up, E) || !qmatvec_q8_supported(w->type_shexp_down, FS))
            return false;
        if (w->rb_shexp_gate_up != qt_row_size(w->type_shexp_gate_up, E) ||
            w->rb_shexp_down != qt_row_size(w->type_shexp_down, FS))
            return false;
    }
    // the flattened vectors of the launches stay within int
    const long long big = (long long)T * (w->n_expert_used + 1) * std::max(E, FE);
    return big < (1LL << 30) && (long long)T * w->n_expert < (1LL << 30);
}

Layout layout(const purhie_moe_weights *w, int T, char *base) {
    Layout L;
    const int E = w->n_embd, FE = w->n_ff_exp, NE = w->n_expert, NU = w->n_expert_used;
    const int FS = has_shexp(w) ? w->n_ff_shexp : 0;
    L.slot = T == 1 && slot_form(w);
    L.grouped = !L.slot && T >= GROUP_MIN_T;
    L.ns = L.slot ? NU + 1 : NU;
    if (L.grouped) {
        L.tile = std::min({qmatvec_id_batch_tile(w->type_gate_up, FE, E), qmatvec_id_batch_tile(w->type_down, E, FE)});
        // 128-entry tiles build each expert's weight planes half as often as 64-entry ones: they win where an
        // expert's mean entry count m fills as many 128-slots as 64-slots (m in (56, 128], (192, 256], ...: config 5's
        // 76 entries 1570 -> 1481 us) and lose where they pad more (config 4's mixed-quant 152 entries: 699 -> 751 us)
        if (L.tile > 64) {
            const double m = (double)T * NU / NE;
            if (m <= 56.0 || std::ceil(m / 128.0) * 128.0 > std::ceil(m / 64.0) * 64.0) L.tile = 64;
        }
        L.max_tiles = gpu_moe_max_tiles(T, NU, NE, L.tile);
    }
    L.qx_k = (int)round256((long long)T * L.ns * FE);
    L.qs_k = FS ? (int)round256((long long)T * FS) : 0;
    size_t off = 0;
    auto take = [&](size_t n) {
        char *p = base ? base + off : nullptr;
        off += (n + 255) & ~(size_t)255;
        return p;
    };
    L.logits = (float *)take((size_t)T * NE * 4);
    if (w->type_router == QT_F16 || w->type_router == QT_BF16) L.xh = (uint16_t *)take((size_t)T * E * 2);
    L.ids = (int32_t *)take((size_t)T * L.ns * 4);
    L.wts = (float *)take((size_t)T * NU * 4);
    L.sg = (float *)take((size_t)T * 4);
    L.g = (float *)take((size_t)T * L.ns * FE * 4);
    L.u = (float *)take((size_t)T * L.ns * FE * 4);
    L.down = (float *)take((size_t)T * L.ns * E * 4);
    L.qx = take(qmatvec_q8_bytes(L.qx_k));
    if (L.grouped) {
        L.tok = (int32_t *)take((size_t)T * NU * 4);
        L.pair = (int32_t *)take((size_t)T * NU * 4);
        L.ntiles = (int32_t *)take(4);
        L.te = (int32_t *)take((size_t)L.max_tiles * 4);
        L.ts = (int32_t *)take((size_t)L.max_tiles * 4);
        L.tn = (int32_t *)take((size_t)L.max_tiles * 4);
    }
    if (FS && !L.slot) {
        L.ffg = (float *)take((size_t)T * FS * 4);
        L.ffu = (float *)take((size_t)T * FS * 4);
        L.sact = (float *)take((size_t)T * FS * 4);
        L.shout = (float *)take((size_t)T * E * 4);
        L.qs = take(qmatvec_q8_bytes(L.qs_k));
    }
    L.bytes = off;
    return L;
}

// scratch's address on the current device, looked up with hipGetSymbolAddress on the first call with that device
// current and kept per device (each GPU holds its own copy of the array at its own address). The array's name is a
// host-side stand-in, never passed to a kernel or a copy.
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch[MAX_DEVICES];

hipError_t scratch_ptr(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return hipSuccess;
}

}  // namespace

extern "C" {

size_t purhie_moe_workspace_bytes(const purhie_moe_weights *w, int T) {
    if (!valid(w, T)) return 0;
    return layout(w, T, nullptr).bytes;
}

int purhie_moe_shared_as_slot(const purhie_moe_weights *w, int T) { return valid(w, T) && T == 1 && slot_form(w); }

hipError_t purhie_moe_ffn(const purhie_moe_weights *w, const float *xn, const qmatvec_q8 *q8_xn, int T, float *out,
                          void *ws, size_t ws_bytes, hipStream_t stream) {
    if (!valid(w, T) || !xn || !q8_xn || !out || !ws || ((uintptr_t)ws & 255)) return hipErrorInvalidValue;
    if ((long long)T * w->n_embd > q8_xn->max_k) return hipErrorInvalidValue;
    const Layout L = layout(w, T, (char *)ws);
    if (ws_bytes < L.bytes) return hipErrorInvalidValue;
    const int E = w->n_embd, FE = w->n_ff_exp, NE = w->n_expert, NU = w->n_expert_used;
    const bool sh = has_shexp(w);
    qmatvec_q8 qx, qs;
    qmatvec_q8_bind(&qx, L.qx, L.qx_k);
    if (!qt_vec_dot_q8k(w->type_down)) qx.qK = nullptr;  // (a Q8_0-activation down never reads the Q8_K side: the
                                                          // SwiGLU launch then skips it)
    hipError_t e;
#define PQ_TRY(call)                       \
    do {                                   \
        if ((e = (call)) != hipSuccess) return e; \
    } while (0)

    // router logits [T][NE]
    if (qmatvec_q8_supported(w->type_router, E))
        PQ_TRY(qmatvec_launch_q8_batch(w->type_router, w->router, w->rb_router, q8_xn, L.logits, NE, NE, E, T, stream));
    else
        PQ_TRY(qmatvec_launch_batch_h(w->type_router, w->router, w->rb_router, xn, L.xh, L.xh ? (size_t)T * E * 2 : 0,
                                      L.logits, NE, E, T, stream));
    // a few tokens without a shared expert: the routing runs inside the expert gate / up launch
    // (qmatvec_launch_q8_id_pair_routed: gpu_moe_router's ids and weights bit for bit, one launch fewer)
    const bool routed = !L.grouped && !L.slot && !sh;
    if (!routed)
        PQ_TRY(gpu_moe_router(L.logits, xn, sh ? w->shexp_gate : nullptr, L.ids, L.wts,
                              sh && w->shexp_gate ? L.sg : nullptr, NE, NU, E, T, stream, L.ns));
    const float *sg = sh && w->shexp_gate ? L.sg : nullptr;

    // the expert down matvec reads SwiGLU(g, u) quantized in its own kernel where the type allows (the same bits
    // as gpu_swiglu's quantization and the plain launch: one launch fewer). The fused launch also needs the tile
    // kernel's alignment (matrices 16-byte aligned); where it refuses a shape (hipErrorInvalidDeviceFunction,
    // before anything runs) the two launches below run instead.
    bool fuse = !L.grouped && qmatvec_q8_id_swiglu_supported(w->type_down, FE);
    auto fused = [&](const void *Wx, float *dst, int ns, int Tn) -> hipError_t {
        const hipError_t r = qmatvec_launch_q8_id_swiglu(w->type_down, w->down_exps, Wx, w->rb_down, L.ids, ns, L.g,
                                                         L.u, dst, E, FE, Tn, stream);
        if (r == hipErrorInvalidDeviceFunction) fuse = false;
        return r == hipErrorInvalidDeviceFunction ? hipSuccess : r;
    };
    if (L.slot) {  // src/qwen_model.cpp:1105-1134: one token, the shared expert as slot NU (id -1)
        PQ_TRY(qmatvec_launch_q8_id_x(w->type_gate_up, w->gate_exps, w->up_exps, w->gate_shexp, w->up_shexp,
                                      w->rb_gate_up, L.ids, L.ns, 0, q8_xn, L.g, L.u, FE, E, 1, stream));
        if (fuse) PQ_TRY(fused(w->down_shexp, L.down, L.ns, 1));
        if (!fuse) {
            PQ_TRY(gpu_swiglu(L.g, L.u, nullptr, L.ns * FE, &qx, stream));  // (the quantized form only)
            PQ_TRY(qmatvec_launch_q8_id_x(w->type_down, w->down_exps, nullptr, w->down_shexp, nullptr, w->rb_down,
                                          L.ids, L.ns, 1, &qx, L.down, nullptr, E, FE, 1, stream));
        }
        return gpu_moe_combine(L.down, L.wts, L.down + (size_t)NU * E, sg, out, NU, E, 1, stream);
    }

    // src/qwen_model.cpp:1137-1166. Grouped, with a down projection that reads Q8_0: SwiGLU and its quantization in
    // the gate / up GEMM's epilogue (the same bits as gpu_swiglu's, one launch and the g / u round trip fewer)
    bool swiglu_done = false;
    if (L.grouped) {
        PQ_TRY(gpu_moe_group(L.ids, T, NU, NE, L.tile, L.tok, L.pair, L.ntiles, L.te, L.ts, L.tn, stream));
        if (!qx.qK && qmatvec_q8_id_batch_swiglu_supported(w->type_gate_up, FE, E)) {
            PQ_TRY(qmatvec_launch_q8_id_batch_swiglu(w->type_gate_up, w->gate_exps, w->up_exps, w->rb_gate_up, q8_xn,
                                                     &qx, FE, E, L.max_tiles, L.tile, L.ntiles, L.te, L.ts, L.tn,
                                                     L.tok, L.pair, stream));
            swiglu_done = true;
        } else {
            PQ_TRY(qmatvec_launch_q8_id_batch_pair(w->type_gate_up, w->gate_exps, w->up_exps, w->rb_gate_up, q8_xn,
                                                   L.g, L.u, FE, E, L.max_tiles, L.tile, L.ntiles, L.te, L.ts, L.tn,
                                                   L.tok, L.pair, stream));
        }
    } else if (routed) {
        PQ_TRY(qmatvec_launch_q8_id_pair_routed(w->type_gate_up, w->gate_exps, w->up_exps, w->rb_gate_up, L.logits, NE,
                                                L.ids, L.wts, NU, q8_xn, L.g, L.u, FE, E, T, stream));
    } else {
        PQ_TRY(qmatvec_launch_q8_id_pair(w->type_gate_up, w->gate_exps, w->up_exps, w->rb_gate_up, L.ids, NU, 0, q8_xn,
                                         L.g, L.u, FE, E, T, stream));
    }
    if (sh) {
        const int FS = w->n_ff_shexp;
        PQ_TRY(qmatvec_launch_q8_batch(w->type_shexp_gate_up, w->gate_shexp, w->rb_shexp_gate_up, q8_xn, L.ffg, FS, FS,
                                       E, T, stream));
        PQ_TRY(qmatvec_launch_q8_batch(w->type_shexp_gate_up, w->up_shexp, w->rb_shexp_gate_up, q8_xn, L.ffu, FS, FS,
                                       E, T, stream));
    }
    if (fuse) PQ_TRY(fused(nullptr, L.down, NU, T));
    if (!fuse) {
        if (!swiglu_done) PQ_TRY(gpu_swiglu(L.g, L.u, nullptr, T * NU * FE, &qx, stream));
        if (L.grouped)
            PQ_TRY(qmatvec_launch_q8_id_batch(w->type_down, w->down_exps, w->rb_down, &qx, L.down, E, FE, L.max_tiles,
                                              L.tile, L.ntiles, L.te, L.ts, L.tn, L.pair, L.pair, stream));
        else
            PQ_TRY(qmatvec_launch_q8_id(w->type_down, w->down_exps, w->rb_down, L.ids, NU, 1, &qx, L.down, E, FE, T,
                                        stream));
    }
    if (!sh) return gpu_moe_combine(L.down, L.wts, nullptr, nullptr, out, NU, E, T, stream);

    const int FS = w->n_ff_shexp;
    qmatvec_q8_bind(&qs, L.qs, L.qs_k);
    if (!qt_vec_dot_q8k(w->type_shexp_down)) qs.qK = nullptr;
    PQ_TRY(gpu_swiglu(L.ffg, L.ffu, L.sact, T * FS, &qs, stream));
    PQ_TRY(qmatvec_launch_q8_batch(w->type_shexp_down, w->down_shexp, w->rb_shexp_down, &qs, L.shout, E, E, FS, T,
                                   stream));
    return gpu_moe_combine(L.down, L.wts, L.shout, sg, out, NU, E, T, stream);
#undef PQ_TRY
}

hipError_t purhie_moe_ffn_noalloc(const purhie_moe_weights *w, const float *xn, const qmatvec_q8 *q8_xn, int T,
                                  float *out, hipStream_t stream) {
    if (!valid(w, T) || layout(w, T, nullptr).bytes > PURHIE_MOE_SCRATCH_BYTES) return hipErrorInvalidValue;
    void *ws = nullptr;
    const hipError_t e = scratch_ptr(&ws);
    if (e != hipSuccess) return e;
    return purhie_moe_ffn(w, xn, q8_xn, T, out, ws, PURHIE_MOE_SCRATCH_BYTES, stream);
}

int purhie_moe_debug_regions(const purhie_moe_weights *w, int T, purhie_moe_regions *r) {
    if (!r || !valid(w, T)) return -1;
    char *const base = (char *)(uintptr_t)256;  // (any aligned base: the offsets are relative to it)
    const Layout L = layout(w, T, base);
    auto off = [&](const void *p) { return p ? (long long)((const char *)p - base) : -1LL; };
    const bool sh = has_shexp(w);
    const bool swiglu_gemm = L.grouped && !qt_vec_dot_q8k(w->type_down) &&
                             qmatvec_q8_id_batch_swiglu_supported(w->type_gate_up, w->n_ff_exp, w->n_embd);
    const bool fused = !L.grouped && qmatvec_q8_id_swiglu_supported(w->type_down, w->n_ff_exp);
    *r = purhie_moe_regions{off(L.ids), off(L.wts), sh && w->shexp_gate ? off(L.sg) : -1, off(L.g), off(L.u),
                            off(L.qx), off(L.down), off(L.shout), off(L.qs), L.ns, L.qx_k, L.qs_k, L.slot ? 1 : 0,
                            L.grouped ? 1 : 0, swiglu_gemm ? 0 : 1, fused ? 0 : 1};
    return 0;
}

}  // extern "C"
