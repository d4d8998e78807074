"""GPU parity of the legacy activation x FP4 GEMM (include/gemm_act_fp4.h) on the reference's own test
construction (tests/actfp4_verify.cpp:30-100: an LCG from 55, A uniform in [-2, 2) as fp16, Codebook10 codes,
UE4M3 scale bytes whose fp4_common.h value lies in [0.1, 1]) against the oracle's double-precision restatement
of the same products: fp32 accumulation keeps the error near 1e-6 of sum |a w| (the reference's GPU rounds each
16-value partial sum to fp16 and is tested at rtol 0.01, atol 0.01 sqrt(K)); and the float-scale (Q4_1 layout)
path against a numpy restatement. The oracle's restatement is pinned on the CPU (test_oracle.py:
test_gemm_act_fp4_closed_forms: numpy matmul of an independently decoded weight, and closed forms)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CB = [0, 1, 2, 3, 4, 6, 8, 10, 0, -1, -2, -3, -4, -6, -8, -10]


class LCG:
    def __init__(self, seed):
        self.s = seed

    def next(self):
        self.s = (self.s * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.s

    def f(self, lo, hi):
        return np.float32(lo + np.float32((self.next() >> 8) / float(1 << 24)) * np.float32(hi - lo))

    def i(self, n):
        return (self.next() >> 8) % n


def ue4m3_common(b):
    e, m = (b >> 3) & 15, b & 7
    raw = m / 512.0 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 8)
    return np.float32(raw * 0.5)


def make(M, N, K, seed=55):
    g = LCG(seed)
    A = np.array([g.f(-2.0, 2.0) for _ in range(M * K)], np.float32).astype(np.float16).reshape(M, K)
    pool = [b for b in range(256) if 0.1 <= ue4m3_common(b) <= 1.0]
    W = np.zeros((N, K // 2), np.uint8)
    S = np.zeros((N, K // 16), np.uint8)
    for n in range(N):
        for s in range(K // 16):
            S[n, s] = pool[g.i(len(pool))]
            for i in range(16):
                k = 16 * s + i
                nib = g.i(16)  # a random codebook entry, stored by its canonical nibble
                W[n, k >> 1] |= nib << ((k & 1) * 4)
    return A, W, S


def run(M, N, K, A, W, S=None, F=None):
    import torch
    from purhie_amd import qmatvec as Q
    L = Q.lib()
    L.gemm_act_fp4_launch.restype = C.c_int
    L.gemm_act_fp4_launch.argtypes = [C.c_void_p] * 5 + [C.c_int] * 3 + [C.c_void_p]
    d = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dA, dW, dS, dF = d(A.view(np.uint16)), d(W), d(S), d(F)
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    ptr = lambda t: None if t is None else C.c_void_p(t.data_ptr())
    assert L.gemm_act_fp4_launch(ptr(dA), ptr(dW), ptr(dS), ptr(dF), ptr(out), M, N, K, None) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("M,N,K", [(16, 16, 16), (37, 29, 48), (64, 96, 256), (130, 70, 512)])
def test_ue4m3_path(oracle, M, N, K):
    A, W, S = make(M, N, K)
    got = run(M, N, K, A, W, S)
    want = oracle.gemm_act_fp4(A.view(np.uint16), W, S, M, N, K)
    wd = np.array([[CB[(W[n, k >> 1] >> ((k & 1) * 4)) & 15] * ue4m3_common(int(S[n, k // 16])) for k in range(K)]
                   for n in range(N)], np.float32).astype(np.float16).astype(np.float64)
    mag = np.abs(A.astype(np.float64)) @ np.abs(wd).T
    assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-6)
    assert np.all(np.abs(got - want) <= 0.01 * np.sqrt(K) + 0.01 * np.abs(want))  # the reference's own bound


@pytest.mark.parametrize("M,N,K", [(20, 33, 64), (64, 64, 256)])
def test_float_scale_path(M, N, K):
    A, W, _ = make(M, N, K, seed=77)
    rng = np.random.default_rng(3)
    F = np.stack([rng.uniform(0.01, 0.2, (N, K // 32)), rng.uniform(-0.05, 0.05, (N, K // 32))], -1).astype(np.float32)
    got = run(M, N, K, A, W, F=F)
    codes = np.array([[CB[(W[n, k >> 1] >> ((k & 1) * 4)) & 15] for k in range(K)] for n in range(N)], np.float64)
    sc = np.repeat(F[:, :, 0].astype(np.float64), 32, axis=1)
    mn = np.repeat(F[:, :, 1].astype(np.float64), 32, axis=1)
    wd = (codes * sc + mn).astype(np.float32).astype(np.float16).astype(np.float64)
    want = A.astype(np.float64) @ wd.T
    mag = np.abs(A.astype(np.float64)) @ np.abs(wd).T
    assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-6)


def test_argument_errors():
    from purhie_amd import qmatvec as Q
    L = Q.lib()
    L.gemm_act_fp4_launch.restype = C.c_int
    L.gemm_act_fp4_launch.argtypes = [C.c_void_p] * 5 + [C.c_int] * 3 + [C.c_void_p]
    assert L.gemm_act_fp4_launch(None, None, None, None, None, 16, 16, 16, None) == 1  # hipErrorInvalidValue
