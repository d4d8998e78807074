"""The split-Q8_0 copy of a float matrix and its matvec (qmatvec_q8_0s_source_supported, qmatvec_quantize_rows_q8_0,
qmatvec_launch_q8_0s; reference src/qmatvec.cpp:369-390, src/matvec_q.hip:3550-3602):
- the copy bit for bit against the oracle's Q8_0 encoder (pinned to the compiled reference's qz_quantize, which is
  ggml's quantize_row_q8_0_ref: d = fp16(amax / 127), q = roundf(x / d) with the fp32 d), for F32, F16 and BF16
  rows, the 34-byte blocks split into values [N][K] and scales [N][K / 32];
- the matvec within 1e-5 * sum |w x| of the oracle's Q8_0 x Q8_0 matvec on the same blocks and activation (the
  reference's criterion, tests/matvec_verify.cpp:117-145);
- the reference's error codes."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
F32, F16, BF16 = 0, 1, 30


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    return qmatvec


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def p(t):
    return C.c_void_p(t.data_ptr())


def source(t, seed, N, K):
    """N x K rows of type t, and the float values they hold"""
    w = synth.gaussian(seed, N * K, 0, 0.05).reshape(N, K)
    w[:, ::61] *= 9.0  # uneven block maxima
    if t == F32:
        return w.view(np.uint8).reshape(N, -1), w
    if t == F16:
        h = w.astype(np.float16)
        return h.view(np.uint8).reshape(N, -1), h.astype(np.float32)
    u = w.view(np.uint32)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return b.view(np.uint8).reshape(N, -1), (b.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("t", (F32, F16, BF16))
@pytest.mark.parametrize("N,K", [(300, 256), (97, 2560), (8, 8192)])
def test_copy_and_matvec(Q, oracle, t, N, K):
    import torch
    L = Q.lib()
    assert L.qmatvec_q8_0s_source_supported(t, K) == 1
    Wb, wf = source(t, 7 + N + K, N, K)
    qs = torch.full((N, K), 99, dtype=torch.int8, device="cuda")
    d = torch.zeros((N, K // 32), dtype=torch.int16, device="cuda")
    assert L.qmatvec_quantize_rows_q8_0(t, p(dev(Wb)), Wb.shape[1], N, K, p(qs), p(d), None) == 0
    blocks = oracle.quantize(8, wf).reshape(N, K // 32, 34)
    want_d = blocks[:, :, :2].copy().view(np.int16).reshape(N, K // 32)
    want_q = blocks[:, :, 2:].copy().view(np.int8).reshape(N, K)
    assert np.array_equal(host(qs), want_q)
    assert np.array_equal(host(d), want_d)
    # the matvec on a quantized activation
    x = synth.gaussian(70 + K, K)
    q = Q.Q8(K)
    Q.quantize(dev(x), K, q)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_q8_0s(p(qs), p(d), q.ref, p(y), N, K, None) == 0
    act = oracle.quantize_act(x, False)
    _, ref, mag = oracle.matvec(8, blocks.reshape(N, -1), N, K, act)
    err = np.abs(host(y).astype(np.float64) - ref) / (mag + 1e-30)
    assert err.max() <= TOL, f"max rel err {err.max():.3g}"


def test_error_codes(Q):
    import torch
    L = Q.lib()
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    y = torch.zeros(64, dtype=torch.float32, device="cuda")
    assert [L.qmatvec_q8_0s_source_supported(t, 256) for t in (0, 1, 30, 8, 12)] == [1, 1, 1, 0, 0]
    assert L.qmatvec_q8_0s_source_supported(0, 320) == 0                        # K % 256
    assert L.qmatvec_quantize_rows_q8_0(8, p(buf), 34 * 8, 4, 256, p(buf), p(buf), None) == 98
    assert L.qmatvec_quantize_rows_q8_0(0, p(buf), 4 * 256 + 4, 4, 256, p(buf), p(buf), None) == 1  # row bytes
    assert L.qmatvec_quantize_rows_q8_0(0, p(buf), 4 * 256, 4, 256, C.c_void_p(buf.data_ptr() + 8), p(buf),
                                        None) == 1                              # qs not 16-byte aligned
    q = Q.Q8(256)
    assert L.qmatvec_launch_q8_0s(p(buf), p(buf), q.ref, p(y), 4, 512, None) == 1  # K > max_k
    assert L.qmatvec_launch_q8_0s(p(buf), p(buf), q.ref, p(y), 4, 128, None) == 1  # K % 256
