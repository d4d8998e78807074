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
    assert [lib.qt_vec_dot_q8k(t) for t in (8, 12, 13, 14, 23, 39, 40, 100, 101)] == [0, 1, 1, 1, 1, 0, 0, 0, 0]


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


# every function of the reference's C headers for this path (src/qmatvec.h:17-199, src/quant_types.h:19-72,
# src/quantize.h:21-45, the producer and MoE part of src/gpu_ops.h, src/gguf_mmap.h:15-121; qmatvec_q8_outputs
# and gpu_moe_max_tiles are header inlines there and here)
REFERENCE_SURFACE = (
    "qmatvec_init qmatvec_free qmatvec_supported qmatvec_launch qmatvec_launch_bf16f qmatvec_launch_batch "
    "qmatvec_launch_batch_h qmatvec_half_supported qmatvec_round_half qmatvec_launch_batch_hx qmatvec_set_prefill "
    "qmatvec_prefill qmatvec_set_prefill_fp32 qmatvec_q8_0s_source_supported qmatvec_quantize_rows_q8_0 "
    "qmatvec_launch_q8_0s qmatvec_q8_bytes qmatvec_q8_bind qmatvec_q8_supported qmatvec_quantize qmatvec_launch_q8 "
    "qmatvec_launch_q8_pair qmatvec_q8_lr_supported qmatvec_launch_q8_lr qmatvec_q8_few_supported "
    "qmatvec_launch_q8_multi qmatvec_launch_q8_multi_t qmatvec_launch_q8_batch qmatvec_launch_q8_id "
    "qmatvec_launch_q8_id_pair qmatvec_launch_q8_id_x qmatvec_launch_id qmatvec_id_batch_tile "
    "qmatvec_q8_id_batch_supported qmatvec_launch_q8_id_batch qmatvec_id_batch_f_supported "
    "qmatvec_launch_id_batch_f qmatvec_set_out_scale qmatvec_drop_out_scales "
    "qt_get_traits qt_row_size qt_to_float qt_vec_dot_q8k qt_fp16_to_fp32 qt_bf16_to_fp32 "
    "qz_supported qz_quantize qz_quantize_im qz_quantize_fp8_blocks qz_fp8_e4m3_to_fp32 qz_row_q8_0 "
    "qz_row_rocmfp4 qz_row_rocmfp4_fast qz_fp32_to_fp16 qz_fp32_to_bf16 "
    # src/gpu_ops.h:20-29,36-48,76: the matvec inputs' producers and the MoE glue
    "gpu_add_rmsnorm gpu_swiglu gpu_moe_router gpu_moe_combine gpu_moe_combine_scaled gpu_moe_group "
    # src/gguf_mmap.h:15-121: the GGUF reader
    "gguf_mmap_open gguf_mmap_close gguf_mmap_get_tensor gguf_n_tensors gguf_tensor_name gguf_tensor_type "
    "gguf_tensor_ne gguf_tensor_dims gguf_tensor_block_size gguf_tensor_type_size gguf_tensor_row_size "
    "gguf_tensor_offset gguf_tensor_nbytes gguf_tensor_nbytes_pad gguf_n_kv gguf_kv_key gguf_kv_type "
    "gguf_kv_get_u8 gguf_kv_get_i8 gguf_kv_get_u16 gguf_kv_get_i16 gguf_kv_get_u32 gguf_kv_get_i32 "
    "gguf_kv_get_f32 gguf_kv_get_u64 gguf_kv_get_i64 gguf_kv_get_f64 gguf_alignment gguf_data_offset "
    "gguf_version gguf_arch gguf_vocab_name gguf_tokenizer_type gguf_pre_type gguf_vocab_size gguf_head_count "
    "gguf_head_count_kv gguf_context_length gguf_embedding_length gguf_block_count gguf_arch_int gguf_arch_float "
    "gguf_kv_str_val gguf_kv_get_string_array gguf_free_string_array gguf_kv_get_array gguf_find_kv "
    "gguf_kv_get_added_tokens gguf_get_tensor_ptr gguf_map_base gguf_n_maps gguf_map_at gguf_remap "
    "gguf_tensor_source gguf_tensor_split gguf_set_tensor_staged gguf_file_path gguf_file_identity "
    "gguf_type_is_self_contained").split()


def test_library_exports_the_reference_surface():
    """an engine built against the reference's headers links: every function they declare is exported"""
    lib = C.CDLL(LIB)
    missing = [n for n in REFERENCE_SURFACE if not hasattr(lib, n)]
    assert not missing, missing
    declared = set(declared_functions())
    assert not [n for n in REFERENCE_SURFACE if n not in declared]


def test_float_path_entries_report_unsupported():
    """the float-activation, split-Q8_0 and low-rank entries answer as the reference does for a missing kernel
    (*_supported 0, launches hipErrorInvalidDeviceFunction, 98, without touching their pointers) for types and shapes
    outside this path (Q4_0, 2; the low-rank entry's ROCmFP4_FAST-only K % 128 <= 1024), and report support for the
    rest"""
    lib = C.CDLL(LIB)
    assert lib.qmatvec_supported(2) == 0
    assert [lib.qmatvec_supported(t) for t in (0, 1, 30, 8, 12, 13, 14, 23, 39, 40, 100, 101)] == [1] * 12
    assert [lib.qmatvec_id_batch_f_supported(t) for t in (0, 1, 30, 8, 12, 100)] == [1] * 6
    assert lib.qmatvec_half_supported(1, None, C.c_size_t(0), 64, 256, 64) == 0
    assert [lib.qmatvec_q8_0s_source_supported(t, 256) for t in (0, 1, 30, 8)] == [1, 1, 1, 0]
    assert lib.qmatvec_q8_0s_source_supported(0, 320) == 0
    assert [lib.qmatvec_q8_lr_supported(t, 384) for t in (101, 100, 12)] == [1, 0, 0]
    assert lib.qmatvec_q8_lr_supported(101, 1152) == 0
    assert lib.qmatvec_id_batch_f_supported(2) == 0
    assert lib.qmatvec_launch(2, None, C.c_size_t(0), None, None, 64, 256, None) == 98
    assert lib.qmatvec_launch_batch(2, None, C.c_size_t(0), None, None, 64, 256, 4, None) == 98
    assert lib.qmatvec_launch_id(2, None, C.c_size_t(0), None, 8, 0, None, None, 64, 256, 1, None) == 98
    assert lib.qmatvec_quantize_rows_q8_0(8, None, C.c_size_t(0), 4, 256, None, None, None) == 98
    assert lib.qmatvec_launch_q8_lr(100, None, C.c_size_t(0), None, 4, 384, C.c_float(1.0), None, 4, None) == 98


def test_fp8_e4m3_decoder(oracle):
    """qz_fp8_e4m3_to_fp32 over all 256 codes: the OCP e4m3fn closed form (bias 7, exponent field 0
    subnormal m 2^-9, S.1111.111 NaN, no infinities), and the compiled reference where it is built"""
    import numpy as np
    L = C.CDLL(LIB)
    L.qz_fp8_e4m3_to_fp32.restype = C.c_float
    L.qz_fp8_e4m3_to_fp32.argtypes = [C.c_uint8]
    got = np.array([L.qz_fp8_e4m3_to_fp32(v) for v in range(256)], np.float32)
    for v in range(256):
        e, m, s = (v >> 3) & 15, v & 7, -1.0 if v & 0x80 else 1.0
        if v & 0x7F == 0x7F:
            assert np.isnan(got[v]) and np.signbit(got[v]) == bool(v & 0x80)
        else:
            assert got[v] == s * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)), v
    assert got[0x7E] == 448.0 and got[0x08] == 2.0 ** -6 and got[0x01] == 2.0 ** -9
    if oracle.ref_available():
        R = oracle.ref()
        R.qz_fp8_e4m3_to_fp32.restype = C.c_float
        R.qz_fp8_e4m3_to_fp32.argtypes = [C.c_uint8]
        want = np.array([R.qz_fp8_e4m3_to_fp32(v) for v in range(256)], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
