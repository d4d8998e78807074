"""GPU parity of the weight encoders (include/quantize.h) against the oracle's restatement of the reference's
CPU encoders (itself pinned bit for bit to the compiled reference and to tests/golden/): every byte equal,
through the host entry point (qz_quantize), the device entry point (qz_quantize_device), re-encoding from
another type, and the one-row functions."""
import os

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu
TYPES = (8, 12, 13, 14, 23, 39, 40, 100, 101)
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    return qmatvec


def rows(seed, n, K):
    """N(0, 0.02) rows, N(0, 1) with outliers, all-zero, constant, tiny, sparse, NaN / Inf rows"""
    x = synth.gaussian(seed, n * K, 0, 0.02).reshape(n, K)
    x[1] = synth.with_outliers(synth.gaussian(seed + 1, K), seed + 2, 0.01, 20.0)
    x[2] = 0.0
    x[3] = 0.37
    x[4] = synth.gaussian(seed + 3, K, 0, 1e-6)
    x[5, 1::7] = 0.0
    x[6, 5] = np.nan
    x[7, 40] = np.inf
    x[7, 300 % K] = -np.inf
    return x.astype(np.float32)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("K", [256, 2560])
def test_encode_host_matches_oracle(Q, oracle, t, K):
    x = rows(700 + t + K, 24, K)
    got = Q.encode(t, x, K)
    assert np.array_equal(got, oracle.quantize(t, x))


@pytest.mark.parametrize("t", TYPES)
def test_encode_golden(Q, t):
    g = dict(np.load(os.path.join(GOLD, f"enc_{t}.npz"), allow_pickle=False))
    assert np.array_equal(Q.encode(t, g["x"], int(g["K"])), g["bytes"])


@pytest.mark.parametrize("t", TYPES)
def test_encode_device_matches_oracle(Q, oracle, t):
    import torch
    N, K = 1000, 1024
    x = synth.gaussian(710 + t, N * K, 0, 0.02).reshape(N, K)
    y = torch.zeros(N * Q.row_size(t, K), dtype=torch.uint8, device="cuda")
    Q.encode_device(t, torch.from_numpy(x).cuda(), y, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().reshape(N, -1), oracle.quantize(t, x))


def test_encode_mxfp4_exponent_rounding_points(Q, oracle):
    """blocks whose maximum lies at or a few units below a power of two, where log2f may round up to the integer
    and the E8M0 exponent with it: the device encoder equals the oracle (itself checked against the compiled
    reference at the same points)"""
    rows = []
    for k in range(-30, 20):
        for ulps in range(6):
            amax = (np.float32(2.0 ** k).view(np.uint32) - np.uint32(ulps)).view(np.float32)
            x = np.clip(synth.gaussian(1000 + 8 * k + ulps, 32, 0, 0.3), -0.9, 0.9).astype(np.float32) * amax
            x[7] = amax
            rows.append(x)
    x = np.stack(rows).astype(np.float32)
    assert np.array_equal(Q.encode(39, x, 32), oracle.quantize(39, x))


@pytest.mark.parametrize("src_t,dst_t", [(1, 100), (30, 12), (8, 101), (100, 8), (12, 14), (14, 13), (1, 40),
                                         (40, 39)])
def test_reencode_from_other_type(Q, oracle, src_t, dst_t):
    K = 512
    x = synth.gaussian(720 + src_t, 8 * K, 0, 0.02).reshape(8, K)
    if src_t == 1:
        src = x.astype(np.float16)
        fl = src.astype(np.float32)
    elif src_t == 30:
        src = (x.view(np.uint32) >> 16).astype(np.uint16)
        fl = (src.astype(np.uint32) << 16).view(np.float32)
    else:
        src = oracle.quantize(src_t, x)
        fl = oracle.to_float(src_t, src, K)
    got = Q.encode(dst_t, src, K, src_type=src_t)
    assert np.array_equal(got, oracle.quantize(dst_t, fl))


def test_row_functions_and_copy(Q, oracle):
    import ctypes as C
    x = synth.gaussian(730, 1024, 0, 0.02)
    for t, fn in ((8, "qz_row_q8_0"), (100, "qz_row_rocmfp4"), (101, "qz_row_rocmfp4_fast")):
        out = np.zeros(Q.row_size(t, 1024), np.uint8)
        getattr(Q.lib(), fn)(x.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), 1024)
        assert np.array_equal(out, oracle.quantize(t, x.reshape(1, -1))[0])
    b = oracle.quantize(12, x.reshape(4, 256))
    assert np.array_equal(Q.encode(12, b, 256, src_type=12), b)  # same type: a copy
