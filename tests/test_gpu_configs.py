"""The benchmark's shapes checked at their real sizes:
- config 2 at batch 4 (the MTP-verify width) on its own matrices: gate and up 9728 x 2560 in one launch and down
  2560 x 9728, four tokens, through both decode kernel families, each output within the reference's tolerance of
  the oracle (|y - y_ref| <= 1e-5 sum |w x|, tests/matvec_verify.cpp:8,142);
- the mixed-quant MoE layer (Q4_K gate / up, Q6_K down experts, a Q8_0 router) at config 4's sizes (hidden 2048,
  128 experts of FFN 768, top-8) for a 2427-token prompt and one token: a sample of the prompt's tokens and the
  single token against the oracle's composition of the same steps (router on the same logits, each expert's gate /
  up, SwiGLU, re-quantization and down, the combine), and every sampled prompt row bit-identical to the same token
  in a 16-token batch (a token's result does not depend on the batch it is grouped in).
Weights come from the library's GPU encoder (its bytes are the oracle's, tests/test_gpu_encode.py), copied to the
host for the oracle."""
import numpy as np
import pytest

from purhie_amd import synth
from tests import moe_stages, parity

pytestmark = pytest.mark.gpu
TOL = 1e-5


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


@pytest.fixture(params=["tile", "wave"])
def kpath(request):
    from purhie_amd import qmatvec
    prev = qmatvec.decode_path(1 if request.param == "tile" else 0)
    yield request.param
    qmatvec.decode_path(prev)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def encoded(Q, t, N, K, seed, sd=0.02):
    """N x K ~N(0, sd) weights encoded as type t on the GPU: (device bytes, host bytes)"""
    import torch
    src = synth.gaussian_torch(torch, seed, N * K, 0.0, sd).reshape(N, K)  # synth.gaussian(seed, N K, 0, sd)
    out = torch.empty((N, Q.row_size(t, K)), dtype=torch.uint8, device="cuda")
    step = max(1, (64 << 20) // (4 * K))
    for r0 in range(0, N, step):
        n = min(step, N - r0)
        Q.encode_device(t, src[r0:r0 + n], out[r0:r0 + n], n, K)
    return out, host(out)


def test_config2_batch4(Q, oracle, kpath):
    import torch
    t, N1, K1, N2, K2, T = 12, 9728, 2560, 2560, 9728, 4
    (gd, gh), (ud, uh), (dd, dh) = (encoded(Q, t, N1, K1, 0xC2001), encoded(Q, t, N1, K1, 0xC2002),
                                    encoded(Q, t, N2, K2, 0xC2003))
    x = synth.gaussian(0xC2004, T * K1).reshape(T, K1)
    h = synth.gaussian(0xC2005, T * K2).reshape(T, K2)
    qx, qh = Q.Q8(T * K1), Q.Q8(T * K2)
    Q.quantize(dev(x.reshape(-1)), T * K1, qx)
    Q.quantize(dev(h.reshape(-1)), T * K2, qh)
    yg, yu = (torch.zeros((T, N1), device="cuda") for _ in range(2))
    yd = torch.zeros((T, N2), device="cuda")
    Q.launch_q8_multi_t(t, [gd, ud], [N1, N1], [yg, yu], qx, K1, T)
    Q.launch_q8_batch(t, dd, qh, yd, N2, N2, K2, T)
    got = {"gate": host(yg), "up": host(yu), "down": host(yd)}
    for i in range(T):
        ax = oracle.quantize_act(x[i], True)
        ah = oracle.quantize_act(h[i], True)
        for name, W, N, K, a in (("gate", gh, N1, K1, ax), ("up", uh, N1, K1, ax), ("down", dh, N2, K2, ah)):
            want, ref, mag = oracle.matvec(t, W, N, K, a)
            parity.check(f"config 2 batch 4 {name} ({kpath})", got[name][i], want, mag, ref, TOL)


E, FE, NE, NU = 2048, 768, 128, 8  # config 4's sizes
T_PROMPT = 2427
SAMPLE = (0, 1, 2, 3, 100, 511, 512, 1000, 1234, 2047, 2048, 2300, 2420, 2424, 2425, 2426)


class Mixed:
    """the mixed-quant layer: Q4_K gate / up, Q6_K down experts, Q8_0 router, no shared expert"""

    def __init__(self, M, Q, seed):
        self.gate_d, self.gate = encoded(Q, 12, NE * FE, E, seed + 1)
        self.up_d, self.up = encoded(Q, 12, NE * FE, E, seed + 2)
        self.down_d, self.down = encoded(Q, 14, NE * E, FE, seed + 3)
        self.router_d, self.router = encoded(Q, 8, NE, E, seed + 4, 0.05)
        w = M.MoeWeights()
        w.n_embd, w.n_ff_exp, w.n_expert, w.n_expert_used = E, FE, NE, NU
        w.type_gate_up, w.type_down = 12, 14
        w.gate_exps, w.up_exps, w.down_exps = (self.gate_d.data_ptr(), self.up_d.data_ptr(),
                                               self.down_d.data_ptr())
        w.rb_gate_up, w.rb_down = Q.row_size(12, E), Q.row_size(14, FE)
        w.type_router, w.router, w.rb_router = 8, self.router_d.data_ptr(), Q.row_size(8, E)
        self.w = w

    def run(self, M, Q, x, keep_ws=False):
        import torch
        T = x.shape[0]
        xd = dev(x)
        q = Q.Q8(((T * E + 255) // 256) * 256)
        Q.quantize(xd.reshape(-1), T * E, q)
        ws = torch.empty(M.workspace_bytes(self.w, T), dtype=torch.uint8, device="cuda")
        out = torch.full((T, E), float("nan"), dtype=torch.float32, device="cuda")
        M.ffn(self.w, xd, q, T, out, ws)
        return (host(out), host(ws)) if keep_ws else host(out)

    def logits(self, Q, x):
        """the router logits as the layer computes them (the same launch, a Q8_0 matvec / GEMM)"""
        import torch
        T = x.shape[0]
        q = Q.Q8(((T * E + 255) // 256) * 256)
        Q.quantize(dev(x.reshape(-1)), T * E, q)
        y = torch.zeros((T, NE), device="cuda")
        Q.launch_q8_batch(8, self.router_d, q, y, NE, NE, E, T)
        return host(y)

    def oracle(self, oracle, x, logits):
        T = x.shape[0]
        ids, wts = oracle.moe_router(logits, NU)
        down = np.zeros((T, NU, E), np.float32)
        for i in range(T):
            a = oracle.quantize_act(x[i], True)
            for j in range(NU):
                e = ids[i, j]
                g = oracle.matvec(12, self.gate[e * FE:(e + 1) * FE], FE, E, a, False)[0]
                u = oracle.matvec(12, self.up[e * FE:(e + 1) * FE], FE, E, a, False)[0]
                hq = oracle.quantize_act(oracle.swiglu(g, u), True)
                down[i, j] = oracle.matvec(14, self.down[e * E:(e + 1) * E], E, FE, hq, False)[0]
        return oracle.moe_combine(down, wts)


def close(got, want, what):
    scale = np.abs(want).max(axis=1, keepdims=True) + 1e-30
    err = (np.abs(got - want) / scale).max()
    assert err <= 2e-3, f"{what}: max error {err:.3g} of the row maximum"


@pytest.fixture(scope="module")
def mixed(M, Q):
    return Mixed(M, Q, 0xC4000)


def test_config4_mixed_prompt(M, Q, oracle, mixed):
    x = synth.gaussian(0xC4100, T_PROMPT * E).reshape(T_PROMPT, E)
    got, ws = mixed.run(M, Q, x, keep_ws=True)
    assert np.isfinite(got).all()
    # the call's own stages on its own inputs: routing and combine of every token bit for bit, the down
    # projections of the sampled tokens within 1e-5 sum |w x|
    moe_stages.check(M, oracle, mixed.w, x, mixed.logits(Q, x), got, ws, mixed.down, 14, NU, rows=SAMPLE)
    del ws
    xs = x[list(SAMPLE)]
    # prefill mode (qmatvec_set_prefill): every batch takes the GEMMs, as the 2427-token call does, so a token's
    # router logits and expert outputs do not depend on the batch
    Q.lib().qmatvec_set_prefill(1)
    try:
        logits = mixed.logits(Q, xs)
        small = mixed.run(M, Q, xs)
    finally:
        Q.lib().qmatvec_set_prefill(0)
    # the sampled tokens against the oracle, on the router logits the layer's own launch gives them
    want = mixed.oracle(oracle, xs, logits)
    close(got[list(SAMPLE)], want, "config 4 mixed, 2427-token prompt")
    # the same tokens as a 16-token batch (the grouped form too): the same bits
    assert np.array_equal(got[list(SAMPLE)].view(np.uint32), small.view(np.uint32))


def test_config4_mixed_one_token(M, Q, oracle, mixed):
    x = synth.gaussian(0xC4200, E).reshape(1, E)
    got, ws = mixed.run(M, Q, x, keep_ws=True)
    moe_stages.check(M, oracle, mixed.w, x, mixed.logits(Q, x), got, ws, mixed.down, 14, NU)
    want = mixed.oracle(oracle, x, mixed.logits(Q, x))
    close(got, want, "config 4 mixed, one token")
