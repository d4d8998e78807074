"""The low-rank up projection (qmatvec_q8_lr_supported, qmatvec_launch_q8_lr; reference src/qmatvec.cpp:467-479,
src/matvec_q.hip:2107-2135): y = W x for one token with x = SiLU(lo * scale) zero-padded from n to K values and
quantized to Q8_0 inside the kernel, over ROCmFP4_FAST weights.
- bit for bit the composition the reference names: SwiGLU(lo * scale, 1) quantized by gpu_swiglu, then
  qmatvec_launch_q8, on both decode kernels (the tile kernel where K is whole units, the per-wave kernel else);
- the composition's activation within one quantization step of the oracle's (SiLU in float32 through numpy's exp,
  the reference's Q8_0 quantizer), and its matvec within 1e-5 * sum |w x| of the oracle's on that activation;
- the reference's error codes."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu

FAST = 101
TOL = 1e-5


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    yield qmatvec
    qmatvec.decode_path(1)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def p(t):
    return C.c_void_p(t.data_ptr())


@pytest.mark.parametrize("path", (1, 0))
@pytest.mark.parametrize("N,K,n", [(1000, 384, 320), (777, 512, 500), (64, 1024, 1024), (300, 128, 77), (40, 256, 0)])
def test_same_bits_as_composition(Q, oracle, path, N, K, n):
    import torch
    from purhie_amd import moe as M
    L = Q.lib()
    prev = Q.decode_path(path)
    try:
        W = oracle.quantize(FAST, synth.gaussian(11 + K + n, N * K, 0, 0.02).reshape(N, K))
        Wd = dev(W)
        lo = synth.gaussian(33 + n, max(n, 1))[:n] * 4.0
        scale = np.float32(0.37)
        y = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
        lod = dev(lo if n else np.zeros(1, np.float32))
        assert L.qmatvec_q8_lr_supported(FAST, K) == 1
        assert L.qmatvec_launch_q8_lr(FAST, p(Wd), W.shape[1], p(lod), n, K, C.c_float(scale), p(y), N, None) == 0
        # the composition: SwiGLU(g, 1) with g = lo scale (fp32 products, as the kernel forms them), then the matvec
        g = np.zeros(K, np.float32)
        g[:n] = lo.astype(np.float32) * scale
        q8 = Q.Q8(((K + 255) // 256) * 256)
        out = torch.empty(K, dtype=torch.float32, device="cuda")
        M.swiglu(dev(g), dev(np.ones(K, np.float32)), out, K, q8)
        yc = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
        Q.launch_q8(FAST, Wd, q8, yc, N, K)
        got, want = host(y), host(yc)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (path, N, K, n)
        # the composition against the oracle
        v = q8.views(K)
        q0, d0 = host(v["q0"]), host(v["d0"])
        s = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
        act = oracle.quantize_act(s, False)
        assert np.abs(q0.astype(np.int32) - act["q"].astype(np.int32)).max() <= 1
        assert np.allclose(d0, act["d"], rtol=1e-3, atol=0)
        _, ref, mag = oracle.matvec(FAST, W, N, K, dict(q=q0, d=d0, s0=act["s0"]))
        err = np.abs(got.astype(np.float64) - ref) / (mag + 1e-30)
        assert err.max() <= TOL, f"max rel err {err.max():.3g}"
    finally:
        Q.decode_path(prev)


def test_error_codes(Q):
    import torch
    L = Q.lib()
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    y = torch.zeros(64, dtype=torch.float32, device="cuda")
    rb = 17 * 384 // 32
    assert [L.qmatvec_q8_lr_supported(t, 384) for t in (101, 100, 8)] == [1, 0, 0]
    assert [L.qmatvec_q8_lr_supported(101, k) for k in (128, 1024, 1152, 200)] == [1, 1, 0, 0]
    assert L.qmatvec_launch_q8_lr(100, p(buf), 18 * 12, p(buf), 10, 384, C.c_float(1.0), p(y), 8, None) == 98
    assert L.qmatvec_launch_q8_lr(101, p(buf), rb, p(buf), 385, 384, C.c_float(1.0), p(y), 8, None) == 1  # n > K
    assert L.qmatvec_launch_q8_lr(101, p(buf), rb + 4, p(buf), 10, 384, C.c_float(1.0), p(y), 8, None) == 1
    assert L.qmatvec_launch_q8_lr(101, C.c_void_p(buf.data_ptr() + 2), rb, p(buf), 10, 384, C.c_float(1.0), p(y), 8,
                                  None) == 1                                           # W not 4-byte aligned
