"""The expert down matvec with the SwiGLU launch folded in (qmatvec_launch_q8_id_swiglu): bit for bit the output of
gpu_swiglu (with its fused Q8_0 quantization) followed by qmatvec_launch_q8_id with x_per_slot = 1 (reference
src/qwen_model.cpp:1117-1131 runs those two launches), for every Q8_0-activation type, with an id of -1 selecting
the extra matrix, per-expert output scales, and several tokens; the K-quants and misaligned K are refused."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu


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
    return None if t is None else C.c_void_p(t.data_ptr())


@pytest.mark.parametrize("t,N,K", [(100, 2048, 768), (101, 1024, 1536), (8, 512, 1024), (39, 768, 2048),
                                   (40, 2048, 768)])
@pytest.mark.parametrize("T", [1, 3])
def test_fused_equals_two_launches(Q, oracle, t, N, K, T):
    import torch
    from purhie_amd import moe as M
    L = Q.lib()
    E, n_used = 16, 8
    W = dev(oracle.quantize(t, synth.gaussian(10 + t, E * N * K, 0, 0.02).reshape(E * N, K)))
    Wx = dev(oracle.quantize(t, synth.gaussian(11 + t, N * K, 0, 0.02).reshape(N, K)))
    rb = Q.row_size(t, K)
    rng = np.random.default_rng(12 + t + T)
    ids = np.stack([rng.permutation(E)[:n_used] for _ in range(T)]).astype(np.int32)
    ids[0, 3] = -1  # the extra matrix (a shared expert as slot)
    g = synth.gaussian(13 + T, T * n_used * K, 0, 2.0).reshape(T * n_used, K)
    u = synth.gaussian(14 + T, T * n_used * K).reshape(T * n_used, K)
    g[1, ::17] = 0.0
    g[2, :] = 0.0  # an all-zero block row: d = 0
    gd, ud, idd = dev(g), dev(u), dev(ids)
    assert L.qmatvec_q8_id_swiglu_supported(t, K) == 1
    # the two launches: SwiGLU with its quantization, then the expert matvec (the extra matrix for slot (0, 3))
    h = torch.zeros(T * n_used * K, device="cuda")
    q = Q.Q8(((T * n_used * K + 255) // 256) * 256)
    assert M.lib().gpu_swiglu(p(gd), p(ud), p(h), T * n_used * K, q.ref, None) == 0
    y2 = torch.full((T * n_used, N), float("nan"), device="cuda")
    assert L.qmatvec_launch_q8_id_swiglu(t, p(W), p(Wx), rb, p(idd), n_used, p(gd), p(ud), p(y2), N, K, T, None) == 0
    y3 = torch.full((T * n_used, N), float("nan"), device="cuda")
    assert L.qmatvec_launch_q8_id_x(t, p(W), None, p(Wx), None, rb, p(idd), n_used, 1, q.ref, p(y3), None, N, K, T,
                                    None) == 0
    a, b = host(y3), host(y2)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # and the per-expert scales apply as on the two-launch path
    es = torch.tensor([0.5 + 0.125 * i for i in range(E)], dtype=torch.float32).pin_memory()
    owner = C.c_void_p(0x51)
    assert L.qmatvec_set_out_scale(owner, p(W), W.numel(), C.c_void_p(es.data_ptr()), E) == 0
    try:
        assert L.qmatvec_launch_q8_id_swiglu(t, p(W), p(Wx), rb, p(idd), n_used, p(gd), p(ud), p(y2), N, K, T,
                                             None) == 0
        assert L.qmatvec_launch_q8_id_x(t, p(W), None, p(Wx), None, rb, p(idd), n_used, 1, q.ref, p(y3), None, N,
                                        K, T, None) == 0
        assert np.array_equal(host(y3).view(np.uint32), host(y2).view(np.uint32))
    finally:
        L.qmatvec_drop_out_scales(owner)


def test_refused(Q):
    import torch
    L = Q.lib()
    z = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    f = torch.zeros(1 << 16, device="cuda")
    ids = torch.zeros(8, dtype=torch.int32, device="cuda")
    assert L.qmatvec_q8_id_swiglu_supported(12, 768) == 0      # K-quant: a Q8_K activation
    assert L.qmatvec_q8_id_swiglu_supported(100, 832) == 0     # K % 256
    assert L.qmatvec_launch_q8_id_swiglu(12, p(z), None, Q.row_size(12, 768), p(ids), 8, p(f), p(f), p(f), 16, 768,
                                         1, None) == 98
    assert L.qmatvec_launch_q8_id_swiglu(100, p(z), None, 18 * 24 + 2, p(ids), 8, p(f), p(f), p(f), 16, 768, 1,
                                         None) == 1  # row bytes
