"""ctypes mirror of include/moe_ops.h (the fused add + RMSNorm + quantize and SwiGLU + quantize producers, and
the MoE router, grouping and combine of libpurhie_qmv.so), the reference's src/gpu_ops.h entry points, and of
include/moe_layer.h (one MoE FFN per call, the engine's moe_core dispatch). Device buffers are torch tensors; every
call runs the library's HIP kernels (no CPU path)."""
import ctypes as C

import numpy as np

from . import qmatvec as Q

_sigs_done = False


def lib():
    global _sigs_done
    L = Q.lib()
    if not _sigs_done:
        vp, i32 = C.c_void_p, C.c_int
        pq8 = C.POINTER(Q.qmatvec_q8)
        for name, args in {
            "gpu_add_rmsnorm": [vp, vp, vp, vp, vp, i32, i32, C.c_float, pq8, vp],
            "gpu_swiglu": [vp, vp, vp, i32, pq8, vp],
            "gpu_moe_router": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32],
            "gpu_moe_combine": [vp, vp, vp, vp, vp, i32, i32, i32, vp],
            "gpu_moe_combine_scaled": [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp],
            "gpu_moe_group": [vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp],
            "purhie_moe_shared_as_slot": [C.POINTER(MoeWeights), i32],
            "purhie_moe_ffn": [C.POINTER(MoeWeights), vp, pq8, i32, vp, vp, C.c_size_t, vp],
            "purhie_moe_ffn_noalloc": [C.POINTER(MoeWeights), vp, pq8, i32, vp, vp],
        }.items():
            f = getattr(L, name)
            f.restype, f.argtypes = i32, args
        L.purhie_moe_debug_regions.restype = i32
        L.purhie_moe_debug_regions.argtypes = [C.POINTER(MoeWeights), i32, C.POINTER(MoeRegions)]
        L.purhie_moe_workspace_bytes.restype = C.c_size_t
        L.purhie_moe_workspace_bytes.argtypes = [C.POINTER(MoeWeights), i32]
        _sigs_done = True
    return L


class MoeWeights(C.Structure):
    """purhie_moe_weights (include/moe_layer.h)"""
    _fields_ = [("n_embd", C.c_int), ("n_ff_exp", C.c_int), ("n_ff_shexp", C.c_int), ("n_expert", C.c_int),
                ("n_expert_used", C.c_int),
                ("type_gate_up", C.c_int), ("type_down", C.c_int),
                ("gate_exps", C.c_void_p), ("up_exps", C.c_void_p), ("down_exps", C.c_void_p),
                ("rb_gate_up", C.c_size_t), ("rb_down", C.c_size_t),
                ("type_router", C.c_int), ("router", C.c_void_p), ("rb_router", C.c_size_t),
                ("type_shexp_gate_up", C.c_int), ("type_shexp_down", C.c_int),
                ("gate_shexp", C.c_void_p), ("up_shexp", C.c_void_p), ("down_shexp", C.c_void_p),
                ("rb_shexp_gate_up", C.c_size_t), ("rb_shexp_down", C.c_size_t),
                ("shexp_gate", C.c_void_p)]


class MoeRegions(C.Structure):
    """purhie_moe_regions (include/moe_layer.h): byte offsets of the layer's intermediate results in its workspace"""
    _fields_ = [(n, C.c_longlong) for n in ("ids", "wts", "sg", "g", "u", "qx", "down", "shout", "qs")] + \
               [(n, C.c_int) for n in ("ns", "qx_k", "qs_k", "slot", "grouped", "gu_written", "act_written")]


def regions(w, T):
    """purhie_moe_debug_regions: where purhie_moe_ffn(w, T) leaves its intermediate results"""
    r = MoeRegions()
    if lib().purhie_moe_debug_regions(C.byref(w), T, C.byref(r)) != 0:
        raise ValueError("the layer cannot run with these weights")
    return r


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def ffn(w, xn, q8, T, out, ws, stream=None):
    """purhie_moe_ffn: out [T][n_embd] from xn [T][n_embd] and its quantized form q8 (a Q.Q8), ws a device
    uint8 tensor of at least workspace_bytes(w, T) bytes"""
    _check("purhie_moe_ffn", lib().purhie_moe_ffn(C.byref(w), _p(xn), q8.ref, T, _p(out), _p(ws), ws.numel(), stream))


def ffn_noalloc(w, xn, q8, T, out, stream=None):
    """purhie_moe_ffn_noalloc: as ffn, with the library's static per-GPU workspace (SCRATCH_BYTES)"""
    _check("purhie_moe_ffn_noalloc", lib().purhie_moe_ffn_noalloc(C.byref(w), _p(xn), q8.ref, T, _p(out), stream))


SCRATCH_BYTES = 32 << 20  # PURHIE_MOE_SCRATCH_BYTES


def workspace_bytes(w, T):
    return lib().purhie_moe_workspace_bytes(C.byref(w), T)


def _check(fn, rc):
    if rc != 0:
        raise Q.HipError(fn, rc)


def max_tiles(T, n_used, n_expert, tile):
    """gpu_moe_max_tiles (include/moe_ops.h)"""
    n = T * n_used
    return min(n, n_expert + n // tile)


def add_rmsnorm(x_in, y, n, T, eps, add=None, x_out=None, w=None, q8=None, stream=None):
    Q._need(x_in, T * n * 4, "x_in")
    Q._need(y, T * n * 4, "y")
    for t_, what in ((add, "add"), (x_out, "x_out")):
        if t_ is not None:
            Q._need(t_, T * n * 4, what)
    if w is not None:
        Q._need(w, n * 4, "w")
    _check("gpu_add_rmsnorm", lib().gpu_add_rmsnorm(_p(x_in), _p(add), _p(x_out), _p(w), _p(y), n, T, eps,
                                                    None if q8 is None else q8.ref, stream))


def swiglu(g, u, out, n, q8=None, stream=None):
    _check("gpu_swiglu", lib().gpu_swiglu(_p(g), _p(u), _p(out), n, None if q8 is None else q8.ref, stream))


def router(logits, ids, wts, n_expert, n_used, T, x=None, w_shexp=None, sg=None, n=0, ids_stride=0, stream=None):
    _check("gpu_moe_router", lib().gpu_moe_router(_p(logits), _p(x), _p(w_shexp), _p(ids), _p(wts), _p(sg), n_expert,
                                                  n_used, n, T, stream, ids_stride))


def combine(down, wts, out, n_used, n, T, shared=None, sg=None, ids=None, exp_scale=None, stream=None):
    if ids is None and exp_scale is None:
        rc = lib().gpu_moe_combine(_p(down), _p(wts), _p(shared), _p(sg), _p(out), n_used, n, T, stream)
    else:
        rc = lib().gpu_moe_combine_scaled(_p(down), _p(wts), _p(shared), _p(sg), _p(ids), _p(exp_scale), _p(out),
                                          n_used, n, T, stream)
    _check("gpu_moe_combine", rc)


def group(ids, T, n_used, n_expert, tile, stream=None):
    """gpu_moe_group into fresh device buffers; returns them as numpy arrays (n_tiles entries of the tiles)"""
    import torch
    n = T * n_used
    mt = max(1, max_tiles(T, n_used, n_expert, tile))
    z = lambda k: torch.full((k,), -7, dtype=torch.int32, device="cuda")
    tok, pair, nt, te, ts, tn = z(max(n, 1)), z(max(n, 1)), z(1), z(mt), z(mt), z(mt)
    _check("gpu_moe_group", lib().gpu_moe_group(_p(ids), T, n_used, n_expert, tile, _p(tok), _p(pair), _p(nt), _p(te),
                                                _p(ts), _p(tn), stream))
    torch.cuda.synchronize()
    k = int(nt.cpu()[0])
    return dict(n_tiles=k, tok_rows=tok.cpu().numpy()[:n], pair_rows=pair.cpu().numpy()[:n],
                tile_e=te.cpu().numpy()[:k], tile_start=ts.cpu().numpy()[:k], tile_n=tn.cpu().numpy()[:k])
