"""GGUF files: a writer (version 3, the public layout) and a ctypes mirror of include/gguf_mmap.h, the library's
reader (the reference's src/gguf_mmap.h API), its HBM staging and its bind_weight.

Layout written: magic "GGUF", version 3, tensor count, key/value count (u64 each); the key/values (key string,
u32 type, value; strings as u64 length + bytes, arrays as u32 element type + u64 count + elements); the tensor
table (name, u32 n_dims, u64 ne[n_dims], u32 type, u64 offset from the data start); zero padding to the alignment
(general.alignment, default 32); the tensor data, each tensor at an aligned offset."""
import ctypes as C
import os
import struct

import numpy as np

from . import qmatvec as Q

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}
_NP = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32, F32: np.float32,
       BOOL: np.uint8, U64: np.uint64, I64: np.int64, F64: np.float64}


def _s(b: bytes):
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _s(v.encode() if isinstance(v, str) else v)
    if t == ARRAY:
        et, items = v
        if et == STRING:
            return struct.pack("<IQ", et, len(items)) + b"".join(_s(x.encode() if isinstance(x, str) else x)
                                                                 for x in items)
        return struct.pack("<IQ", et, len(items)) + np.asarray(items, dtype=_NP[et]).tobytes()
    return struct.pack(_FMT[t], v)


def write(path, kvs, tensors, alignment=None):
    """kvs: [(key, type, value)] (arrays: (ARRAY, (elem_type, items))); tensors: [(name, ggml_type, ne tuple,
    bytes)]. Writes general.alignment when `alignment` is given. Returns the data offset of every tensor."""
    kvs = list(kvs)
    align = 32 if alignment is None else alignment
    if alignment is not None:
        kvs.append(("general.alignment", U32, alignment))
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs)))
    for k, t, v in kvs:
        out += _s(k.encode()) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, t, ne, data in tensors:
        off = (off + align - 1) // align * align
        offs.append(off)
        out += _s(name.encode()) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        out += struct.pack("<IQ", t, off)
        off += len(data)
    out += b"\0" * ((-len(out)) % align)
    base = len(out)
    for (name, t, ne, data), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)
    return offs


class gguf_weight(C.Structure):
    _fields_ = [("type", C.c_int), ("N", C.c_int), ("K", C.c_int), ("row_bytes", C.c_size_t), ("data", C.c_void_p)]


_bound = set()
_L = None


def lib():
    """the library's reader (host code: it loads without a GPU; only gguf_hbm_stage needs one)"""
    global _L
    if _L is None:
        if not os.path.exists(Q.LIB_PATH):
            raise RuntimeError(f"{Q.LIB_PATH} is missing: build it with __graft_entry__.build()")
        _L = C.CDLL(Q.LIB_PATH)
    return bind(_L)


def bind(L):
    """set the argument and result types of every gguf_* entry point a CDLL has (this library's, or another
    build of the same API)"""
    if id(L) not in _bound:
        vp, i64, sz = C.c_void_p, C.c_int64, C.c_size_t
        for name, res, args in [
            ("gguf_mmap_open", vp, [C.c_char_p]), ("gguf_mmap_close", None, [vp]),
            ("gguf_get_tensor_ptr", vp, [vp, C.c_char_p, C.POINTER(sz)]),
            ("gguf_mmap_get_tensor", vp, [vp, C.c_char_p, C.POINTER(sz)]),
            ("gguf_n_tensors", i64, [vp]), ("gguf_tensor_name", C.c_char_p, [vp, i64]),
            ("gguf_tensor_type", C.c_int, [vp, i64]), ("gguf_tensor_ne", C.POINTER(i64), [vp, i64]),
            ("gguf_tensor_dims", C.c_uint8, [vp, i64]), ("gguf_tensor_block_size", sz, [vp, i64]),
            ("gguf_tensor_type_size", sz, [vp, i64]), ("gguf_tensor_row_size", sz, [vp, i64]),
            ("gguf_tensor_offset", C.c_uint64, [vp, i64]), ("gguf_tensor_nbytes", sz, [vp, i64]),
            ("gguf_tensor_nbytes_pad", sz, [vp, i64]), ("gguf_n_kv", i64, [vp]),
            ("gguf_kv_key", C.c_char_p, [vp, i64]), ("gguf_kv_type", C.c_int, [vp, i64]),
            ("gguf_kv_str_val", C.c_char_p, [vp, i64]), ("gguf_find_kv", i64, [vp, C.c_char_p]),
            ("gguf_alignment", sz, [vp]), ("gguf_data_offset", sz, [vp]), ("gguf_version", C.c_uint32, [vp]),
            ("gguf_arch", C.c_char_p, [vp]), ("gguf_vocab_name", C.c_char_p, [vp]),
            ("gguf_tokenizer_type", C.c_char_p, [vp]), ("gguf_pre_type", C.c_char_p, [vp]),
            ("gguf_vocab_size", i64, [vp]), ("gguf_head_count", i64, [vp]), ("gguf_head_count_kv", i64, [vp]),
            ("gguf_context_length", i64, [vp]), ("gguf_embedding_length", i64, [vp]),
            ("gguf_block_count", i64, [vp]), ("gguf_arch_int", i64, [vp, C.c_char_p, i64]),
            ("gguf_arch_float", C.c_float, [vp, C.c_char_p, C.c_float]),
            ("gguf_kv_get_string_array", C.c_int32, [vp, C.c_char_p, C.POINTER(C.POINTER(C.c_char_p)),
                                                     C.POINTER(sz)]),
            ("gguf_kv_get_added_tokens", C.c_int32, [vp, C.c_char_p, C.POINTER(C.POINTER(C.c_char_p)),
                                                     C.POINTER(sz)]),
            ("gguf_kv_get_array", C.c_int32, [vp, C.c_char_p, C.POINTER(C.c_int32), C.POINTER(vp), C.POINTER(sz)]),
            ("gguf_map_base", vp, [vp, C.POINTER(sz)]), ("gguf_n_maps", C.c_int, [vp]),
            ("gguf_map_at", vp, [vp, C.c_int, C.POINTER(sz)]), ("gguf_remap", C.c_int, [vp, vp, sz]),
            ("gguf_tensor_source", vp, [vp, i64]), ("gguf_tensor_split", C.c_int, [vp, i64]),
            ("gguf_set_tensor_staged", None, [vp, i64, vp]), ("gguf_file_path", C.c_char_p, [vp, C.c_int]),
            ("gguf_file_identity", C.c_int, [vp, C.c_int, C.POINTER(C.c_uint64)]),
            ("gguf_type_is_self_contained", C.c_int, [C.c_int]),
            ("gguf_hbm_bytes", sz, [vp, vp]), ("gguf_hbm_stage", C.c_int, [vp, vp, sz, vp, vp]),
            ("gguf_bind_weight", C.c_int, [vp, C.c_char_p, C.POINTER(gguf_weight)]),
        ]:
            if hasattr(L, name):
                f = getattr(L, name)
                f.restype, f.argtypes = res, args
        for t in ("u8", "i8", "u16", "i16", "u32", "i32", "f32", "u64", "i64", "f64"):
            ct = {"u8": C.c_uint8, "i8": C.c_int8, "u16": C.c_uint16, "i16": C.c_int16, "u32": C.c_uint32,
                  "i32": C.c_int32, "f32": C.c_float, "u64": C.c_uint64, "i64": C.c_int64, "f64": C.c_double}[t]
            f = getattr(L, f"gguf_kv_get_{t}")
            f.restype, f.argtypes = C.c_int32, [vp, i64, C.POINTER(ct)]
        _bound.add(id(L))
    return L


class Model:
    """an open GGUF file (gguf_mmap_open); closed by close() or the context manager"""

    def __init__(self, path, L=None):
        self.L = lib() if L is None else bind(L)
        self.h = self.L.gguf_mmap_open(str(path).encode())
        if not self.h:
            raise OSError(f"gguf_mmap_open refused {path}")

    def close(self):
        if self.h:
            self.L.gguf_mmap_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def tensor(self, name):
        n = C.c_size_t()
        p = self.L.gguf_get_tensor_ptr(self.h, name.encode(), C.byref(n))
        return (p, n.value) if p else (None, 0)

    def names(self):
        return [self.L.gguf_tensor_name(self.h, i).decode() for i in range(self.L.gguf_n_tensors(self.h))]

    def kv_index(self, key):
        return self.L.gguf_find_kv(self.h, key.encode())

    def get(self, getter, key_or_idx):
        idx = key_or_idx if isinstance(key_or_idx, int) else self.kv_index(key_or_idx)
        f = getattr(self.L, f"gguf_kv_get_{getter}")
        out = f.argtypes[2]._type_()
        rc = f(self.h, idx, C.byref(out))
        return rc, out.value

    def hbm_stage(self, dev_buf, keep=None, stream=None):
        """stage the tensors (keep: per-index flags, None = all) into a device buffer (a torch uint8 tensor)"""
        k = None if keep is None else np.ascontiguousarray(keep, dtype=np.uint8)
        need = self.L.gguf_hbm_bytes(self.h, None if k is None else k.ctypes.data)
        rc = self.L.gguf_hbm_stage(self.h, C.c_void_p(dev_buf.data_ptr()), dev_buf.numel(),
                                   None if k is None else k.ctypes.data, stream)
        return rc, need

    def hbm_bytes(self, keep=None):
        k = None if keep is None else np.ascontiguousarray(keep, dtype=np.uint8)
        return self.L.gguf_hbm_bytes(self.h, None if k is None else k.ctypes.data)

    def bind_weight(self, name):
        w = gguf_weight()
        rc = self.L.gguf_bind_weight(self.h, name.encode(), C.byref(w))
        return rc, w
