"""The exact ROCmFP4 GEMM on the f8f6f4 matrix core (gemm_f8.hip, qmatvec_debug_gemm_f8f6f4): the measured
alternative to the split GEMM. Its per-16-value integer dots are exact by construction (E4M3 codebook levels, the
activation in two exact 4-bit planes, one pair of instructions per group) and its epilogue is the reference's
(e_w d_x) c per group (src/matvec_q.hip:2566-2973), so every output is checked against the oracle within the
path's bound, 1e-5 sum |w x| (tests/matvec_verify.cpp:8,142), on random block bytes (every code and scale byte),
with partial row and token tiles."""
import numpy as np
import pytest

from purhie_amd import synth
from tests import parity

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K,T", [(256, 1024, 128), (300, 2048, 70), (1000, 512, 257), (128, 5120, 40)])
def test_f8f6f4_gemm_matches_oracle(oracle, N, K, T):
    import torch
    from purhie_amd import qmatvec as Q
    Q.lib()
    t = 100
    rb = Q.row_size(t, K)
    W = (synth.splitmix64(400 + N, N * rb) & np.uint64(0xFF)).astype(np.uint8).reshape(N, rb)
    x = synth.with_outliers(synth.gaussian(401 + T, T * K), 402, 0.001, 20.0).reshape(T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(torch.from_numpy(x.reshape(-1)).cuda(), T * K, q)
    y = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    Q.gemm_f8f6f4(torch.from_numpy(W).cuda(), q, y, N, K, T)
    got = y.cpu().numpy()
    for i in range(T):
        want, ref, mag = oracle.matvec(t, W, N, K, oracle.quantize_act(x[i], False))
        parity.check("f8f6f4 exact GEMM rocmfp4", got[i], want, mag, ref)


def test_f8f6f4_gemm_rejects(oracle):
    import ctypes as C
    import torch
    from purhie_amd import qmatvec as Q
    L = Q.lib()
    q = Q.Q8(1024)
    y = torch.zeros(64 * 64, device="cuda")
    W = torch.zeros((64, Q.row_size(100, 1024)), dtype=torch.uint8, device="cuda")
    p = lambda a: C.c_void_p(a.data_ptr())
    assert L.qmatvec_debug_gemm_f8f6f4(p(W), Q.row_size(100, 1024), q.ref, p(y), 64, 64, 1024, 2, None) == 1  # T K > max_k
    assert L.qmatvec_debug_gemm_f8f6f4(p(W), Q.row_size(100, 1024) + 1, q.ref, p(y), 64, 64, 1024, 1, None) == 1
