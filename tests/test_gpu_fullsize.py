"""The configs at their full sizes: the checks that do not grow with the size.
Config 3: the ROCmFP4 17408 x 5120 prefill GEMM over 2427 tokens (0.1% outliers x20, as the benchmark builds
them): sampled tokens against the oracle within 1e-5 * sum |w x| (the reference's criterion,
tests/matvec_verify.cpp:8,142), and prefill-mode rows independent of how the prompt is cut, bit for bit.
Config 4: 128 ROCmFP4 experts (hidden 2048, FFN 768), top-8, through the one-call MoE layer: one decode token and a
512-token prefill, sampled tokens against the oracle's composition of the same steps on the same router logits."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

from tests import moe_stages

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    yield qmatvec
    qmatvec.lib().qmatvec_set_prefill(0)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def p(t):
    return C.c_void_p(t.data_ptr())


def encoded(Q, t, N, K, seed):
    """N x K ~N(0, 0.02) weights, synth.gaussian(seed, N K, 0, 0.02) made on the device, encoded on the device
    (bit-identical to the oracle's encoder, tests/test_gpu_encode.py)"""
    import torch
    out = torch.empty((N, Q.row_size(t, K)), dtype=torch.uint8, device="cuda")
    step = max(1, (64 << 20) // K)
    for r0 in range(0, N, step):
        n = min(step, N - r0)
        w = synth.gaussian_torch(torch, seed, n * K, 0.0, 0.02, start=r0 * K).reshape(n, K)
        Q.encode_device(t, w, out[r0:r0 + n], n, K)
    return out


def test_config3_prefill_full_size(Q, oracle):
    import torch
    t, N, K, T = 100, 17408, 5120, 2427
    L = Q.lib()
    Wd = encoded(Q, t, N, K, 0x5EED0003)
    W = host(Wd)
    x = synth.with_outliers(synth.gaussian(0x5EED1003, T * K), 0x5EED1103, 0.001, 20.0).reshape(T, K)
    xd = torch.from_numpy(x).cuda()
    q = Q.Q8(T * K)
    Q.quantize(xd.reshape(-1), T * K, q)
    L.qmatvec_set_prefill(1)
    try:
        y = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
        Q.launch_q8_batch(t, Wd, q, y, N, N, K, T)
        full = host(y)
        # a cut of the prompt: tokens 1000 .. 1063 alone give the same bits
        a, b = 1000, 1064
        qa = Q.Q8((b - a) * K)
        Q.quantize(xd[a:b].reshape(-1), (b - a) * K, qa)
        ya = torch.full((b - a, N), float("nan"), dtype=torch.float32, device="cuda")
        Q.launch_q8_batch(t, Wd, qa, ya, N, N, K, b - a)
        assert np.array_equal(host(ya).view(np.uint32), full[a:b].view(np.uint32))
    finally:
        L.qmatvec_set_prefill(0)
    assert np.isfinite(full).all()
    for i in (0, 1, 777, 1500, 2426):
        want, ref, mag = oracle.matvec(t, W, N, K, oracle.quantize_act(x[i], False))
        assert np.all(np.abs(full[i] - want) <= TOL * mag), i
        assert np.all(np.abs(full[i] - ref) <= TOL * mag), i


@pytest.mark.parametrize("T", [1, 512])
def test_config4_moe_full_size(Q, oracle, T):
    import torch
    from purhie_amd import moe as M
    t, NE, NU, H, F = 100, 128, 8, 2048, 768
    gate, up, down = encoded(Q, t, NE * F, H, 0x5EED0004), encoded(Q, t, NE * F, H, 0x5EED0104), \
        encoded(Q, t, NE * H, F, 0x5EED0204)
    rw = synth.gaussian(0x5EED0304, NE * H, 0, 0.05).reshape(NE, H)
    router = torch.from_numpy(rw).cuda()
    w = M.MoeWeights()
    w.n_embd, w.n_ff_exp, w.n_expert, w.n_expert_used = H, F, NE, NU
    w.type_gate_up, w.type_down = t, t
    w.gate_exps, w.up_exps, w.down_exps = gate.data_ptr(), up.data_ptr(), down.data_ptr()
    w.rb_gate_up, w.rb_down = Q.row_size(t, H), Q.row_size(t, F)
    w.type_router, w.router, w.rb_router = 0, router.data_ptr(), 4 * H
    x = synth.gaussian(0x5EED1004 + T, T * H).reshape(T, H)
    xd = torch.from_numpy(x).cuda()
    q = Q.Q8(((T * H + 255) // 256) * 256)
    Q.quantize(xd.reshape(-1), T * H, q)
    ws = torch.empty(M.workspace_bytes(w, T), dtype=torch.uint8, device="cuda")
    out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
    M.ffn(w, xd, q, T, out, ws)
    got = host(out)
    # the router logits as the call computes them (the float decode kernel over the F32 router)
    lg = torch.empty((T, NE), dtype=torch.float32, device="cuda")
    assert Q.lib().qmatvec_launch_batch(0, p(router), 4 * H, p(xd), p(lg), NE, H, T, None) == 0
    logits = host(lg)
    Wg, Wu, Wdn = host(gate), host(up), host(down)
    # the call's own stages on its own inputs (routing and combine bit for bit, the sampled tokens' down projections
    # within 1e-5 sum |w x|); then the whole layer against the oracle's composition as a reading
    moe_stages.check(M, oracle, w, x, logits, got, host(ws), Wdn, t, NU, rows=sorted({0, T // 3, T - 1}))
    for i in sorted({0, T // 3, T - 1}):
        ids, wts = oracle.moe_router(logits[i:i + 1], NU)
        a = oracle.quantize_act(x[i], False)
        dn = np.zeros((1, NU, H), np.float32)
        for j in range(NU):
            e = ids[0, j]
            g = oracle.matvec(t, Wg[e * F:(e + 1) * F], F, H, a, False)[0]
            u = oracle.matvec(t, Wu[e * F:(e + 1) * F], F, H, a, False)[0]
            h = oracle.swiglu(g, u)
            dn[0, j] = oracle.matvec(t, Wdn[e * H:(e + 1) * H], H, F, oracle.quantize_act(h, False), False)[0]
        want = oracle.moe_combine(dn, wts)[0]
        err = np.abs(got[i] - want).max() / (np.abs(want).max() + 1e-30)
        assert err <= 2e-3, (i, err)
