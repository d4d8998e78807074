"""The drop-in boundary without a GPU: the C-ABI library loads and exports every function that
include/*.h declares, and the host-side metadata agrees with the reference's (no compute calls)."""
import ctypes as C
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "purhie_amd", "libpurhie_qmv.so")


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        src = re.sub(r"static inline[^{]*\{.*?\n\}", "", src, flags=re.S)  # header-only helpers
        src = "\n".join(l for l in src.split("\n") if not l.lstrip().startswith("#"))
        src = src.replace('extern "C" {', "")
        for stmt in src.split(";"):
            s = " ".join(stmt.split())
            if not s or s.startswith("typedef") or "(*" in s or s.startswith("#"):
                continue
            m = re.search(r"\b([A-Za-z_]\w*)\s*\([^()]*(\([^()]*\)[^()]*)*\)\s*$", s)
            if m and not s.startswith("enum") and "=" not in s.split("(")[0]:
                names.add(m.group(1))
    return sorted(names)


def test_headers_declare_the_reference_surface():
    names = declared_functions()
    for n in ("qmatvec_init", "qmatvec_quantize", "qmatvec_launch_q8", "qmatvec_launch_q8_multi_t",
              "qmatvec_launch_q8_batch", "qmatvec_launch_q8_id_x", "qmatvec_launch_q8_id_batch", "qt_row_size",
              "qt_to_float", "qt_get_traits", "gpu_swiglu", "gpu_moe_router", "gpu_moe_combine",
              "gpu_moe_combine_scaled", "gpu_moe_group", "qz_supported", "qz_quantize", "qz_quantize_im",
              "qz_row_q8_0", "qz_row_rocmfp4", "qz_row_rocmfp4_fast", "qz_fp32_to_fp16", "qz_fp32_to_bf16",
              "gemm_act_fp4_launch"):
        assert n in names, n


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built")
    lib = C.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in include/*.h but not exported: {missing}"


def test_row_sizes_and_traits_match_reference_metadata():
    lib = C.CDLL(LIB)
    lib.qt_row_size.restype = C.c_size_t
    lib.qt_row_size.argtypes = [C.c_int, C.c_int64]
    lib.qt_vec_dot_q8k.argtypes = [C.c_int]
    # survey row a1's figures (src/quant_types.cpp:586-615 block geometry)
    cases = {(8, 1024): 1088, (12, 2560): 1440, (12, 9728): 5472, (100, 5120): 2880, (100, 2048): 1152,
             (100, 768): 432, (12, 2048): 1152, (14, 1024): 840, (8, 3072): 3264, (101, 4096): 2176,
             (8, 100): 0, (12, 300): 0}
    for (t, k), want in cases.items():
        assert lib.qt_row_size(t, k) == want, (t, k)
    assert [lib.qt_vec_dot_q8k(t) for t in (8, 12, 14, 100, 101)] == [0, 1, 1, 0, 0]


def test_q8_buffer_layout():
    lib = C.CDLL(LIB)
    lib.qmatvec_q8_bytes.restype = C.c_size_t
    # 2 K + 2 (K/32 * 4) + K/256 * 4 + K/16 * 4, every section 16-aligned (src/qmatvec.cpp:397-419)
    assert lib.qmatvec_q8_bytes(4096) == 2 * 4096 + 2 * 512 + 64 + 1024


def test_host_scalar_conversions(oracle):
    """qz_fp32_to_fp16 / qz_fp32_to_bf16 (host functions of the library) against the oracle's binary16
    rounding (pinned exhaustively) and the compiled reference, on random bit patterns and special values"""
    import numpy as np
    L = C.CDLL(LIB)
    L.qz_fp32_to_fp16.restype = L.qz_fp32_to_bf16.restype = C.c_uint16
    L.qz_fp32_to_fp16.argtypes = L.qz_fp32_to_bf16.argtypes = [C.c_float]
    from purhie_amd import synth
    bits = synth.splitmix64(31, 20000).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00001, 0xffc12345, 0x7f800001, 0x477ff000,
                        0x477fefff, 0x38800000, 0x387fffff, 0x33000000, 0x33000001, 0x00000001, 0x3f800000],
                       dtype=np.uint32)
    xs = np.concatenate([bits, special]).view(np.float32)
    want16 = oracle.f32_to_f16(xs)
    got16 = np.array([L.qz_fp32_to_fp16(C.c_float(v)) for v in xs], dtype=np.uint16)
    assert np.array_equal(got16, want16)
    u = xs.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7fffffff) > 0x7f800000
    want_bf = np.where(nan, (u >> 16) | 64, (u + 0x7fff + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    got_bf = np.array([L.qz_fp32_to_bf16(C.c_float(v)) for v in xs], dtype=np.uint16)
    assert np.array_equal(got_bf, want_bf)
    if oracle.ref_available():
        R = oracle.ref()
        R.qz_fp32_to_bf16.restype = C.c_uint16
        R.qz_fp32_to_bf16.argtypes = [C.c_float]
        assert np.array_equal(got_bf, np.array([R.qz_fp32_to_bf16(C.c_float(v)) for v in xs], dtype=np.uint16))
