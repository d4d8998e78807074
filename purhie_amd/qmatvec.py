"""ctypes mirror of the C ABI in include/qmatvec.h and include/quant_types.h (libpurhie_qmv.so).

The reference's interface for this path is the C one (src/qmatvec.h, src/quant_types.h); this module
exposes the same entry points, argument meaning and error behaviour to Python, with torch tensors as
the device buffers (torch is plumbing here: memory and streams). Every call runs the library's HIP
kernels; there is no CPU path, and loading fails loudly when the library is missing.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpurhie_qmv.so")

QT_F32, QT_F16, QT_Q8_0, QT_Q4_K, QT_Q5_K, QT_Q6_K, QT_IQ4_XS, QT_BF16 = 0, 1, 8, 12, 13, 14, 23, 30
QT_MXFP4, QT_NVFP4 = 39, 40
QT_Q4_0_ROCMFP4, QT_Q4_0_ROCMFP4_FAST = 100, 101
KQUANTS = (QT_Q4_K, QT_Q5_K, QT_Q6_K, QT_IQ4_XS)
NAMES = {QT_Q8_0: "q8_0", QT_Q4_K: "q4_K", QT_Q5_K: "q5_K", QT_Q6_K: "q6_K", QT_IQ4_XS: "iq4_xs", QT_Q4_0_ROCMFP4: "q4_0_rocmfp4",
         QT_Q4_0_ROCMFP4_FAST: "q4_0_rocmfp4_fast", QT_MXFP4: "mxfp4", QT_NVFP4: "nvfp4"}
GROUP = {QT_Q8_0: 32, QT_Q4_0_ROCMFP4: 16, QT_Q4_0_ROCMFP4_FAST: 32, QT_Q4_K: 32, QT_Q5_K: 32, QT_Q6_K: 16, QT_IQ4_XS: 32,
         QT_MXFP4: 32, QT_NVFP4: 16}


class HipError(RuntimeError):
    def __init__(self, fn, code):
        super().__init__(f"{fn} returned hipError {code}")
        self.code = code


hipSuccess, hipErrorInvalidValue, hipErrorInvalidDeviceFunction = 0, 1, 98


class qmatvec_q8(C.Structure):
    _fields_ = [("q0", C.c_void_p), ("d0", C.c_void_p), ("qK", C.c_void_p), ("dK", C.c_void_p),
                ("bsK", C.c_void_p), ("s0", C.c_void_p), ("max_k", C.c_int), ("xh", C.c_void_p),
                ("xh_bf16", C.c_int)]


class qt_traits(C.Structure):
    _fields_ = [("type", C.c_int), ("name", C.c_char_p), ("blck_size", C.c_int), ("type_size", C.c_int),
                ("to_float", C.c_void_p), ("verified", C.c_int)]


_lib = None


def lib():
    """the library, loaded once; raises if it has not been built (no fallback exists)"""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "(make -C purhie_amd/csrc); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        vp, i32, sz, i64, ll = C.c_void_p, C.c_int, C.c_size_t, C.c_int64, C.c_longlong
        pq8 = C.POINTER(qmatvec_q8)
        sigs = {
            "qmatvec_init": (i32, [C.c_char_p]),
            "qmatvec_free": (None, []),
            "qmatvec_q8_bytes": (sz, [i32]),
            "qmatvec_q8_bind": (None, [pq8, vp, i32]),
            "qmatvec_q8_supported": (i32, [i32, i32]),
            "qmatvec_q8_few_supported": (i32, [i32, i32, i32]),
            "qmatvec_quantize": (i32, [vp, i32, pq8, vp]),
            "qmatvec_launch_q8": (i32, [i32, vp, sz, pq8, vp, i32, i32, vp]),
            "qmatvec_launch_q8_pair": (i32, [i32, vp, i32, vp, vp, i32, vp, sz, pq8, i32, vp]),
            "qmatvec_launch_q8_multi": (i32, [i32, i32, C.POINTER(vp), C.POINTER(i32), C.POINTER(vp), sz, pq8, i32,
                                              vp]),
            "qmatvec_launch_q8_multi_t": (i32, [i32, i32, C.POINTER(vp), C.POINTER(i32), C.POINTER(vp), sz, pq8, i32,
                                                i32, vp]),
            "qmatvec_launch_q8_batch": (i32, [i32, vp, sz, pq8, vp, ll, i32, i32, i32, vp]),
            "qmatvec_launch_q8_id": (i32, [i32, vp, sz, vp, i32, i32, pq8, vp, i32, i32, i32, vp]),
            "qmatvec_launch_q8_id_pair": (i32, [i32, vp, vp, sz, vp, i32, i32, pq8, vp, vp, i32, i32, i32, vp]),
            "qmatvec_launch_q8_id_pair_routed": (i32, [i32, vp, vp, sz, vp, i32, vp, vp, i32, pq8, vp, vp, i32, i32, i32,
                                                       vp]),
            "qmatvec_launch_q8_id_x": (i32, [i32, vp, vp, vp, vp, sz, vp, i32, i32, pq8, vp, vp, i32, i32, i32, vp]),
            "qmatvec_q8_id_batch_swiglu_supported": (i32, [i32, i32, i32]),
            "qmatvec_launch_q8_id_batch_swiglu": (i32, [i32, vp, vp, sz, pq8, pq8, i32, i32, i32, i32, vp, vp, vp, vp,
                                                        vp, vp, vp]),
            "qmatvec_id_batch_tile": (i32, [i32, i32, i32]),
            "qmatvec_q8_id_batch_supported": (i32, [i32, i32]),
            "qmatvec_launch_q8_id_batch": (i32, [i32, vp, sz, pq8, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp,
                                                 vp]),
            "qmatvec_launch_q8_id_batch_pair": (i32, [i32, vp, vp, sz, pq8, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp,
                                                      vp, vp, vp]),
            "qmatvec_debug_block_dots": (i32, [i32, vp, sz, pq8, vp, i32, i32, vp]),
            "qmatvec_debug_gemm_f8f6f4": (i32, [vp, sz, pq8, vp, i32, i32, i32, i32, vp]),
            "qmatvec_debug_capture": (i32, [vp, sz]),
            "qmatvec_debug_capture_unit": (i32, [i32, i32]),
            "qmatvec_debug_decode_path": (i32, [i32]),
            "qmatvec_set_prefill": (None, [i32]),
            "qmatvec_prefill": (i32, []),
            "qmatvec_set_out_scale": (i32, [vp, vp, sz, vp, i32]),
            "qmatvec_supported": (i32, [i32]),
            "qmatvec_q8_id_swiglu_supported": (i32, [i32, i32]),
            "qmatvec_launch_q8_id_swiglu": (i32, [i32, vp, vp, sz, vp, i32, vp, vp, vp, i32, i32, i32, vp]),
            "qmatvec_launch": (i32, [i32, vp, sz, vp, vp, i32, i32, vp]),
            "qmatvec_launch_id": (i32, [i32, vp, sz, vp, i32, i32, vp, vp, i32, i32, i32, vp]),
            "qmatvec_id_batch_f_supported": (i32, [i32]),
            "qmatvec_q8_0s_source_supported": (i32, [i32, i32]),
            "qmatvec_quantize_rows_q8_0": (i32, [i32, vp, sz, i32, i32, vp, vp, vp]),
            "qmatvec_launch_q8_0s": (i32, [vp, vp, pq8, vp, i32, i32, vp]),
            "qmatvec_q8_lr_supported": (i32, [i32, i32]),
            "qmatvec_launch_q8_lr": (i32, [i32, vp, sz, vp, i32, i32, C.c_float, vp, i32, vp]),
            "qmatvec_launch_id_batch_f": (i32, [i32, vp, sz, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]),
            "qmatvec_launch_bf16f": (i32, [vp, sz, vp, vp, i32, i32, i32, vp]),
            "qmatvec_launch_batch": (i32, [i32, vp, sz, vp, vp, i32, i32, i32, vp]),
            "qmatvec_launch_batch_h": (i32, [i32, vp, sz, vp, vp, sz, vp, i32, i32, i32, vp]),
            "qmatvec_half_supported": (i32, [i32, vp, sz, i32, i32, i32]),
            "qmatvec_round_half": (i32, [i32, vp, vp, ll, vp]),
            "qmatvec_launch_batch_hx": (i32, [i32, vp, sz, vp, vp, i32, i32, i32, vp]),
            "qmatvec_set_prefill_fp32": (None, [i32]),
            "qmatvec_drop_out_scales": (None, [vp]),
            "qt_get_traits": (C.POINTER(qt_traits), [i32]),
            "qt_row_size": (sz, [i32, i64]),
            "qt_to_float": (i32, [i32, vp, vp, i64]),
            "qt_to_float_device": (i32, [i32, vp, vp, i64, vp]),
            "qt_vec_dot_q8k": (i32, [i32]),
            "qt_fp16_to_fp32": (C.c_float, [C.c_uint16]),
            "qz_supported": (i32, [i32]),
            "qz_quantize": (i32, [i32, vp, i32, vp, i64, i64, i32, C.c_char_p, sz]),
            "qz_quantize_im": (i32, [i32, vp, i32, vp, i64, i64, vp, i32, C.c_char_p, sz]),
            "qz_quantize_device": (i32, [i32, vp, vp, i64, i64, vp]),
            "qz_row_q8_0": (None, [vp, vp, i64]),
            "qz_row_rocmfp4": (None, [vp, vp, i64]),
            "qz_row_rocmfp4_fast": (None, [vp, vp, i64]),
            "qz_fp32_to_fp16": (C.c_uint16, [C.c_float]),
            "qz_fp32_to_bf16": (C.c_uint16, [C.c_float]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        if L.qmatvec_init(None) != 0:
            raise RuntimeError("qmatvec_init failed: no HIP device")
        _lib = L
    return _lib


def _check(fn, rc):
    if rc != hipSuccess:
        raise HipError(fn, rc)


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _need(t, nbytes, what):
    """a host-side bound check before a launch: the tensor holds at least nbytes contiguous bytes"""
    have = t.numel() * t.element_size()
    if have < nbytes or not t.is_contiguous():
        raise ValueError(f"{what}: {have} bytes (contiguous: {t.is_contiguous()}), the launch reads or writes {nbytes}")


def row_size(t, k):
    return int(lib().qt_row_size(t, k))


def reads_q8k(t):
    return t in KQUANTS


class Q8:
    """a qmatvec_q8 bound to a device buffer of qmatvec_q8_bytes(max_k) bytes"""

    def __init__(self, max_k, device="cuda"):
        import torch
        assert max_k % 256 == 0
        self.max_k = max_k
        self.mem = torch.zeros(int(lib().qmatvec_q8_bytes(max_k)), dtype=torch.uint8, device=device)
        self.s = qmatvec_q8()
        lib().qmatvec_q8_bind(C.byref(self.s), C.c_void_p(self.mem.data_ptr()), max_k)

    @property
    def ref(self):
        return C.byref(self.s)

    def views(self, k):
        """torch views of the first k values' quantized forms (q0, d0, s0, qK, dK, bsK)"""
        import torch
        base = self.mem.data_ptr()

        def view(ptr, n, dt):
            off = ptr - base
            nbytes = n * torch.empty(0, dtype=dt).element_size()
            return self.mem[off:off + nbytes].view(dt)

        return dict(q0=view(self.s.q0, k, torch.int8), d0=view(self.s.d0, k // 32, torch.float32),
                    s0=view(self.s.s0, k // 32, torch.int32), qK=view(self.s.qK, k, torch.int8),
                    dK=view(self.s.dK, k // 256, torch.float32), bsK=view(self.s.bsK, k // 16, torch.int32))


def quantize(x, K, q, stream=None):
    _need(x, K * 4, "x")
    _check("qmatvec_quantize", lib().qmatvec_quantize(_p(x), K, q.ref, stream))


def launch_q8(t, W, q, y, N, K, stream=None):
    _need(W, N * row_size(t, K), "W")
    _need(y, N * 4, "y")
    _check("qmatvec_launch_q8", lib().qmatvec_launch_q8(t, _p(W), row_size(t, K), q.ref, _p(y), N, K, stream))


def launch_q8_multi_t(t, Ws, Ns, ys, q, K, T, stream=None):
    for w, n_, y_ in zip(Ws, Ns, ys):
        _need(w, n_ * row_size(t, K), "W")
        _need(y_, T * n_ * 4, "y")
    n = len(Ws)
    wa = (C.c_void_p * n)(*[w.data_ptr() for w in Ws])
    na = (C.c_int * n)(*Ns)
    ya = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    _check("qmatvec_launch_q8_multi_t",
           lib().qmatvec_launch_q8_multi_t(t, n, wa, na, ya, row_size(t, K), q.ref, K, T, stream))


def launch_q8_batch(t, W, q, y, ldy, N, K, T, stream=None):
    _need(W, N * row_size(t, K), "W")
    _need(y, ((T - 1) * ldy + N) * 4, "y")
    _check("qmatvec_launch_q8_batch",
           lib().qmatvec_launch_q8_batch(t, _p(W), row_size(t, K), q.ref, _p(y), ldy, N, K, T, stream))


def launch_q8_id_x(t, W, W2, Wx, W2x, ids, n_used, x_per_slot, q, y, y2, N, K, T, stream=None):
    _check("qmatvec_launch_q8_id_x",
           lib().qmatvec_launch_q8_id_x(t, _p(W), _p(W2), _p(Wx), _p(W2x), row_size(t, K), _p(ids), n_used,
                                        x_per_slot, q.ref, _p(y), _p(y2), N, K, T, stream))


class capture:
    """capture mode (qmatvec_debug_capture) for the launches inside the `with` block: the kernels also add every
    integer sum they form into `out` (an int32 device tensor, zeroed here), in the layouts include/qmatvec.h
    gives"""

    def __init__(self, out):
        self.out = out

    def __enter__(self):
        self.out.zero_()
        _check("qmatvec_debug_capture", lib().qmatvec_debug_capture(_p(self.out), self.out.numel()))
        return self.out

    def __exit__(self, *exc):
        lib().qmatvec_debug_capture(None, 0)
        return False


def capture_unit(t, gemm=False):
    """values per captured integer: the decode kernels' scale group, or the GEMM's epilogue unit (0: none)"""
    return lib().qmatvec_debug_capture_unit(t, 1 if gemm else 0)


def decode_path(mode=None):
    """the decode kernels in use: 1 = tile kernels where they take the shape, 0 = per-wave kernels only; sets
    `mode` when given and returns the previous one"""
    return lib().qmatvec_debug_decode_path(-1 if mode is None else mode)


def gemm_f8f6f4(W, q, y, N, K, T, stream=None):
    """qmatvec_debug_gemm_f8f6f4: the exact ROCmFP4 GEMM on the f8f6f4 matrix core, y [T][N]"""
    _check("qmatvec_debug_gemm_f8f6f4",
           lib().qmatvec_debug_gemm_f8f6f4(_p(W), row_size(100, K), q.ref, _p(y), N, N, K, T, stream))


def block_dots(t, W, q, out, N, K, stream=None):
    _check("qmatvec_debug_block_dots",
           lib().qmatvec_debug_block_dots(t, _p(W), row_size(t, K), q.ref, _p(out), N, K, stream))


def to_float_device(t, src, dst, n, stream=None):
    _check("qt_to_float_device", lib().qt_to_float_device(t, _p(src), _p(dst), n, stream))


def to_float_host(t, src, n):
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    rc = lib().qt_to_float(t, src.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), n)
    if rc != 0:
        raise RuntimeError(f"qt_to_float({t}) failed")
    return out


def encode(t, src, ncols, src_type=QT_F32):
    """qz_quantize: host rows (src_type; fp32 by default) -> host bytes of type t, [rows][row_size(t, ncols)]"""
    src = np.ascontiguousarray(src)
    nrows = src.nbytes // row_size(src_type, ncols) if src_type != QT_F32 else src.size // ncols
    out = np.zeros((nrows, row_size(t, ncols)), dtype=np.uint8)
    err = C.create_string_buffer(256)
    rc = lib().qz_quantize(t, out.ctypes.data_as(C.c_void_p), src_type, src.ctypes.data_as(C.c_void_p), nrows, ncols,
                           0, err, 256)
    if rc != 0:
        raise RuntimeError(err.value.decode())
    return out


def encode_device(t, src, dst, nrows, ncols, stream=None):
    """qz_quantize_device: fp32 rows in device memory -> type t rows in device memory"""
    _check("qz_quantize_device", lib().qz_quantize_device(t, _p(dst), _p(src), nrows, ncols, stream))
