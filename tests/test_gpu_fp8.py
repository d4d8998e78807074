"""GPU parity of qz_quantize_fp8_blocks (include/quantize.h): FP8 e4m3fn rows times a float32 scale per
block_rows x block_cols block, encoded as each type, byte for byte against the oracle's encoder applied to the
same products (numpy float32 multiply: one rounding, as src/quantize.cpp:1241-1258), and against the
compiled reference's own qz_quantize_fp8_blocks where it is built."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu


def fp8_values():
    """the 256 e4m3fn codes' values (closed form, NaN for S.1111.111)"""
    out = np.empty(256, np.float32)
    for v in range(256):
        e, m = (v >> 3) & 15, v & 7
        f = np.nan if v & 0x7F == 0x7F else (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
        out[v] = -f if v & 0x80 else f
    return out


@pytest.mark.parametrize("t", (8, 12, 14, 100, 101, 0, 1))
def test_fp8_blocks_encode(oracle, t):
    from purhie_amd import qmatvec as Q
    L = Q.lib()
    rows, cols, br, bc = 300, 512, 128, 128
    codes = (synth.splitmix64(31 + t, rows * cols) % np.uint64(256)).astype(np.uint8)
    codes[codes & 0x7F == 0x7F] = 0x38  # (NaN codes out of the numeric check)
    codes = codes.reshape(rows, cols)
    sc_cols = cols // bc + 1  # a wider scale row than needed, as the argument allows
    scale = (np.abs(synth.gaussian(32 + t, ((rows + br - 1) // br) * sc_cols)) * 0.01 + 1e-4).astype(np.float32)
    scale = scale.reshape(-1, sc_cols)
    vals = fp8_values()[codes] * np.repeat(np.repeat(scale, br, axis=0)[:rows], bc, axis=1)[:, :cols]
    rb = Q.row_size(t, cols)
    out = np.zeros((rows, rb), np.uint8)
    err = C.create_string_buffer(256)
    L.qz_quantize_fp8_blocks.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int,
                                         C.c_int, C.c_int64, C.c_int, C.c_char_p, C.c_size_t]
    rc = L.qz_quantize_fp8_blocks(t, out.ctypes.data, codes.ctypes.data, scale.ctypes.data, rows, cols, br, bc,
                                  sc_cols, 0, err, 256)
    assert rc == 0, err.value
    want = oracle.quantize(t, vals.astype(np.float32))
    assert np.array_equal(out, want.reshape(rows, rb))
    if oracle.ref_available():
        R = oracle.ref()
        R.qz_quantize_fp8_blocks.argtypes = L.qz_quantize_fp8_blocks.argtypes
        ref = np.zeros_like(out)
        assert R.qz_quantize_fp8_blocks(t, ref.ctypes.data, codes.ctypes.data, scale.ctypes.data, rows, cols, br, bc,
                                        sc_cols, 1, err, 256) == 0
        assert np.array_equal(out, ref)


def test_fp8_blocks_bad_arguments():
    from purhie_amd import qmatvec as Q
    L = Q.lib()
    err = C.create_string_buffer(256)
    L.qz_quantize_fp8_blocks.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int,
                                         C.c_int, C.c_int64, C.c_int, C.c_char_p, C.c_size_t]
    b = np.zeros(64, np.uint8)
    s = np.ones(4, np.float32)
    # scale rows narrower than the blocks of a row need
    assert L.qz_quantize_fp8_blocks(8, b.ctypes.data, b.ctypes.data, s.ctypes.data, 1, 64, 1, 16, 3, 0, err, 256) == -1
    assert b"bad arguments" in err.value
