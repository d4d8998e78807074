"""purhie_moe_ffn_noalloc (include/moe_layer.h): the MoE FFN on the library's static per-GPU workspace gives the
bits of purhie_moe_ffn on a caller's workspace, on two calls in a row (the second with fewer tokens, so it runs
on what the first left in the array), for config 4's sizes with ROCmFP4 experts and with Q4_K gate / up, Q6_K
down; a T whose workspace exceeds the array is refused before any launch."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu

E, FE, NE, NU = 2048, 768, 128, 8  # config 4: hidden 2048, 128 experts of FFN 768, top 8


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    return qmatvec


@pytest.fixture(scope="module")
def M():
    from purhie_amd import moe
    moe.lib()
    return moe


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def encoded(Q, t, N, K, seed):
    import torch
    src = synth.gaussian_torch(torch, seed, N * K, 0.0, 0.02).reshape(N, K)
    out = torch.empty((N, Q.row_size(t, K)), dtype=torch.uint8, device="cuda")
    Q.encode_device(t, src, out, N, K)
    return out


def layer(M, Q, t_gu, t_d, seed):
    keep = [encoded(Q, t_gu, NE * FE, E, seed), encoded(Q, t_gu, NE * FE, E, seed + 1),
            encoded(Q, t_d, NE * E, FE, seed + 2), dev(synth.gaussian(seed + 3, NE * E, 0, 0.05))]
    w = M.MoeWeights()
    w.n_embd, w.n_ff_exp, w.n_expert, w.n_expert_used = E, FE, NE, NU
    w.type_gate_up, w.type_down = t_gu, t_d
    w.gate_exps, w.up_exps, w.down_exps = [k.data_ptr() for k in keep[:3]]
    w.rb_gate_up, w.rb_down = Q.row_size(t_gu, E), Q.row_size(t_d, FE)
    w.type_router, w.router, w.rb_router = 0, keep[3].data_ptr(), E * 4
    return w, keep


@pytest.mark.parametrize("t_gu,t_d", [(100, 100), (12, 14)], ids=["rocmfp4", "q4k_q6k"])
def test_noalloc_matches_workspace_form(M, Q, t_gu, t_d):
    import torch
    w, keep = layer(M, Q, t_gu, t_d, 21)
    for T in (24, 5):  # the expert-grouped GEMM form, then the per-token form on the array the first call left
        print(f"noalloc case: types {t_gu}/{t_d}, T {T}", flush=True)
        xd = dev(synth.gaussian(30 + T, T * E).reshape(T, E))
        q = Q.Q8(((T * E + 255) // 256) * 256)
        Q.quantize(xd.reshape(-1), T * E, q)
        nb = M.workspace_bytes(w, T)
        assert 0 < nb <= M.SCRATCH_BYTES
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        want = torch.full((T, E), float("nan"), dtype=torch.float32, device="cuda")
        M.ffn(w, xd, q, T, want, ws)
        got = torch.full((T, E), float("nan"), dtype=torch.float32, device="cuda")
        M.ffn_noalloc(w, xd, q, T, got)
        torch.cuda.synchronize()
        a, b = got.cpu().numpy(), want.cpu().numpy()
        assert np.isfinite(b).all() and np.abs(b).max() > 0
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"T={T}: the static workspace changed the bits"


def test_noalloc_refuses_beyond_the_array(M, Q):
    import torch
    w, keep = layer(M, Q, 100, 100, 41)
    T = 257  # the first token count whose workspace exceeds 32 MiB at these sizes
    assert M.workspace_bytes(w, T) > M.SCRATCH_BYTES >= M.workspace_bytes(w, T - 1)
    xd = torch.zeros((T, E), dtype=torch.float32, device="cuda")
    q = Q.Q8(((T * E + 255) // 256) * 256)
    out = torch.full((T, E), 7.0, dtype=torch.float32, device="cuda")
    rc = M.lib().purhie_moe_ffn_noalloc(C.byref(w), C.c_void_p(xd.data_ptr()), q.ref, T,
                                         C.c_void_p(out.data_ptr()), None)
    assert rc == 1  # hipErrorInvalidValue, nothing launched
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 7.0).all()
