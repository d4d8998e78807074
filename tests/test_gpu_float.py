"""Float activations over F32 / F16 / BF16 weights (qmatvec_launch, _batch, _batch_h, _batch_hx, round_half,
half_supported, launch_bf16f; reference src/qmatvec.h:29-75, src/qmatvec.cpp:255-366, src/matvec_q.hip:700-1075,
3391-3547): every output within 1e-5 * sum |w x| of the oracle's double sum over the activations rounded to the
weight type (the reference's own criterion, tests/matvec_verify.cpp:117-145,147-189); the 16-bit rounding bit for
bit; a token's decode output the same bits alone or in a batch; the GEMM the same bits with the caller's scratch or
without, and for a token alone or inside a batch in prefill mode; the reference's error codes."""
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
    yield qmatvec
    qmatvec.lib().qmatvec_set_prefill(0)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def weights(t, seed, N, K):
    w = synth.gaussian(seed, N * K, 0, 0.05).reshape(N, K)
    if t == F32:
        return w.view(np.uint8)
    if t == F16:
        return w.astype(np.float16).view(np.uint8)
    u = w.view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8)


def acts(seed, T, K):
    x = synth.gaussian(seed, T * K).reshape(T, K)
    x[:, ::97] *= 30.0  # a few large values
    return x


def check(oracle, t, W, N, K, x, got, round=True):
    ref, mag = oracle.matvec_float(t, W, N, K, x, round)
    err = np.abs(got.astype(np.float64) - ref) / (mag + 1e-30)
    assert err.max() <= TOL, f"max rel err {err.max():.3g}"


@pytest.mark.parametrize("t", (F32, F16, BF16))
@pytest.mark.parametrize("N,K", [(4096, 2048), (1000, 5120), (1, 8), (7, 100), (64, 1000)])
def test_decode_matvec(Q, oracle, t, N, K):
    import torch
    L = Q.lib()
    W = weights(t, 10 + N, N, K)
    x = acts(20 + K, 1, K)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch(t, p(dev(W)), W.shape[1], p(dev(x)), p(y), N, K, None) == 0
    check(oracle, t, W, N, K, x, host(y)[None])


@pytest.mark.parametrize("t", (F32, F16, BF16))
def test_decode_batch_same_bits_as_single(Q, oracle, t):
    """below the GEMM threshold a batch runs the decode kernel: each token's row the same bits as alone"""
    import torch
    L = Q.lib()
    N, K, T = 512, 2048, 7
    Wd = dev(weights(t, 31, N, K))
    x = acts(32, T, K)
    y = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_batch(t, p(Wd), Wd.numel() // N, p(dev(x)), p(y), N, K, T, None) == 0
    got = host(y)
    check(oracle, t, host(Wd).reshape(N, -1), N, K, x, got)
    one = torch.empty(N, dtype=torch.float32, device="cuda")
    for i in range(T):
        assert L.qmatvec_launch(t, p(Wd), Wd.numel() // N, p(dev(x[i])), p(one), N, K, None) == 0
        assert np.array_equal(host(one).view(np.uint32), got[i].view(np.uint32)), i


@pytest.mark.parametrize("t", (F16, BF16))
@pytest.mark.parametrize("N,K,T", [(256, 1024, 70), (200, 2048, 130), (1024, 5120, 33), (2048, 2048, 256),
                                   (64, 8, 40), (130, 1000, 129)])
def test_half_gemm(Q, oracle, t, N, K, T):
    """the MFMA GEMM through _batch (the 16-bit copy in a pooled buffer) and _batch_h (in the caller's scratch:
    qmatvec_round_half, then _batch_hx): the same bits, within tolerance of the oracle, and the copy is the
    rounding bit for bit"""
    import torch
    L = Q.lib()
    W = weights(t, 40 + N, N, K)
    Wd = dev(W)
    x = acts(41 + T, T, K)
    xd = dev(x)
    rb = W.shape[1]
    assert L.qmatvec_half_supported(t, p(Wd), rb, N, K, T) == 1
    y1 = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_batch(t, p(Wd), rb, p(xd), p(y1), N, K, T, None) == 0
    xh = torch.empty(T * K, dtype=torch.uint16, device="cuda")
    y2 = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_batch_h(t, p(Wd), rb, p(xd), p(xh), T * K * 2, p(y2), N, K, T, None) == 0
    g1, g2 = host(y1), host(y2)
    assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
    check(oracle, t, W, N, K, x, g1)
    # the 16-bit copy is the rounding, bit for bit
    want = oracle.act_round(t, x).view(np.uint32) >> 16 if t == BF16 else \
        oracle.act_round(t, x).astype(np.float16).view(np.uint16)
    assert np.array_equal(host(xh).reshape(T, K).astype(np.uint32), want.astype(np.uint32))


@pytest.mark.parametrize("t", (F16, BF16))
def test_half_gemm_256_row_tiles(Q, oracle, t):
    """N = 2200 (a partial last row tile), K = 1000 (a partial last stage), T = 2000: enough workgroups for the
    256-row tiles on MI355X's 256 CUs. The fp32-x form the same bits as the scratch form, sampled tokens within
    tolerance of the oracle, and every token's row the same bits as a 40-token launch (128-row tiles) gives it:
    the row tile does not change the summation order."""
    import torch
    L = Q.lib()
    N, K, T = 2200, 1000, 2000
    W = weights(t, 60, N, K)
    Wd = dev(W)
    rb = W.shape[1]
    x = acts(61, T, K)
    assert L.qmatvec_half_supported(t, p(Wd), rb, N, K, T) == 1
    y1 = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_batch(t, p(Wd), rb, p(dev(x)), p(y1), N, K, T, None) == 0
    xh = torch.empty(T * K, dtype=torch.uint16, device="cuda")
    y2 = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_batch_h(t, p(Wd), rb, p(dev(x)), p(xh), T * K * 2, p(y2), N, K, T, None) == 0
    g1, g2 = host(y1), host(y2)
    assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
    sel = np.arange(0, T, 21)
    check(oracle, t, W, N, K, x[sel], g1[sel])
    for a, b in ((0, 40), (1000, 1040), (1960, 2000)):
        part = torch.full((b - a, N), float("nan"), dtype=torch.float32, device="cuda")
        assert L.qmatvec_launch_batch(t, p(Wd), rb, p(dev(x[a:b])), p(part), N, K, b - a, None) == 0
        assert np.array_equal(host(part).view(np.uint32), g1[a:b].view(np.uint32)), (a, b)


@pytest.mark.parametrize("t", (F16, BF16))
def test_round_half_special_values(Q, oracle, t):
    import torch
    L = Q.lib()
    x = np.float32([0.0, -0.0, 1.0, 65504.0, 65520.0, 1e30, -1e30, 6e-8, 1e-40, np.inf, -np.inf, 3.3961e38,
                    1.0000001, 1.00390625, 1.01171875, -2.5, 0.1, 7e4])
    x = np.concatenate([x, synth.gaussian(5, 8 * 1024) * np.float32(1000.0)]).astype(np.float32)
    x = x[: x.size // 8 * 8]
    xh = torch.empty(x.size, dtype=torch.uint16, device="cuda")
    assert L.qmatvec_round_half(t, p(dev(x)), p(xh), x.size, None) == 0
    got = host(xh)
    r = oracle.act_round(t, x)
    if t == BF16:
        want = (r.view(np.uint32) >> 16).astype(np.uint16)
    else:
        with np.errstate(over="ignore"):
            want = r.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # NaN stays NaN
    n = np.full(8, np.nan, np.float32)
    assert L.qmatvec_round_half(t, p(dev(n)), p(xh), 8, None) == 0
    h = host(xh)[:8]
    v = h.view(np.float16).astype(np.float32) if t == F16 else (h.astype(np.uint32) << 16).view(np.float32)
    assert np.isnan(v).all()


@pytest.mark.parametrize("t", (F16, BF16))
def test_prefill_rows_independent_of_batch_cut(Q, oracle, t):
    """prefill mode takes every batch, one token included, to the GEMM: a token's row the same bits however
    the prompt is cut"""
    import torch
    L = Q.lib()
    N, K, T = 320, 1536, 70
    Wd = dev(weights(t, 50, N, K))
    rb = Wd.numel() // N
    x = acts(51, T, K)
    L.qmatvec_set_prefill(1)
    try:
        assert L.qmatvec_half_supported(t, p(Wd), rb, N, K, 1) == 1
        y = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
        assert L.qmatvec_launch_batch(t, p(Wd), rb, p(dev(x)), p(y), N, K, T, None) == 0
        full = host(y)
        for a, b in ((0, 1), (1, 65), (65, 70)):
            part = torch.full((b - a, N), float("nan"), dtype=torch.float32, device="cuda")
            assert L.qmatvec_launch_batch(t, p(Wd), rb, p(dev(x[a:b])), p(part), N, K, b - a, None) == 0
            assert np.array_equal(host(part).view(np.uint32), full[a:b].view(np.uint32)), (a, b)
    finally:
        L.qmatvec_set_prefill(0)
    assert L.qmatvec_half_supported(t, p(Wd), rb, N, K, 1) == 0


def test_bf16f_raw_activations(Q, oracle):
    """qmatvec_launch_bf16f: BF16 weights times the fp32 activations as they are (1 and 5 tokens)"""
    import torch
    L = Q.lib()
    N, K = 768, 2048
    W = weights(BF16, 60, N, K)
    Wd = dev(W)
    for T in (1, 5):
        x = acts(61 + T, T, K)
        y = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
        assert L.qmatvec_launch_bf16f(p(Wd), 2 * K, p(dev(x)), p(y), N, K, T, None) == 0
        check(oracle, BF16, W, N, K, x, host(y), round=False)
        # and not the rounded-activation result (the activations have more than 8 significant bits)
        ref_r, _ = oracle.matvec_float(BF16, W, N, K, x, True)
        assert not np.array_equal(host(y).astype(np.float64), ref_r)


def test_float_error_codes(Q):
    import torch
    L = Q.lib()
    W = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    x = torch.zeros(4096, dtype=torch.float32, device="cuda")
    y = torch.zeros(4096, dtype=torch.float32, device="cuda")
    assert [L.qmatvec_supported(t) for t in (0, 1, 30, 8, 12, 100, 2)] == [1, 1, 1, 1, 1, 1, 0]
    assert L.qmatvec_launch(2, p(W), 18 * 2, p(x), p(y), 4, 64, None) == 98     # no float kernel for Q4_0
    assert L.qmatvec_launch(1, p(W), 2 * 64 + 2, p(x), p(y), 4, 64, None) == 1  # row bytes != 2 K
    assert L.qmatvec_launch_bf16f(p(W), 2 * 64, p(x), p(y), 4, 64, 0, None) == 1  # T < 1
    assert L.qmatvec_half_supported(1, p(W), 2 * 1024, 64, 1024, 31) == 0  # under 32 tokens outside prefill
    assert L.qmatvec_half_supported(1, p(W), 2 * 1024, 63, 1024, 32) == 0  # under 64 rows
    assert L.qmatvec_half_supported(1, p(W), 2 * 1020, 64, 1020, 32) == 0  # K % 8
    assert L.qmatvec_half_supported(0, p(W), 4 * 1024, 64, 1024, 32) == 0  # F32 has no MFMA GEMM
    assert L.qmatvec_half_supported(30, p(W), 2 * 1024, 64, 1024, 32) == 1
    assert L.qmatvec_round_half(1, p(x), C.c_void_p(W.data_ptr() + 2), 64, None) == 1  # misaligned
    assert L.qmatvec_round_half(1, p(x), p(W), 60, None) == 1                          # n % 8
    assert L.qmatvec_round_half(12, p(x), p(W), 64, None) == 98
    assert L.qmatvec_launch_batch_hx(1, p(W), 2 * 1024, p(W), p(y), 64, 1024, 8, None) == 98
