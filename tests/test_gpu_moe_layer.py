"""One MoE FFN per call (purhie_moe_ffn, include/moe_layer.h): the engine's moe_core / moe_core_one /
shared_as_slot (reference src/qwen_model.cpp:1093-1166) over the library's launches. The one-token form with the
shared expert as slot -1 gives the same bits as the plain launch sequence (the reference's claim for its 3-launch
form); every form (slot, per-token matvecs below 8 tokens, expert-grouped GEMMs from 8, no shared expert, F32 /
BF16 / Q8_0 routers) matches the oracle's composition of the same steps (router on the same logits, each expert's
gate / up, SwiGLU, re-quantization and down, the shared expert, the combine); the dispatch rules and argument
checks."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

from tests import moe_stages

pytestmark = pytest.mark.gpu

KQ = (12, 13, 14, 23)


@pytest.fixture(scope="module")
def M():
    from purhie_amd import moe
    moe.lib()
    return moe


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


class Layer:
    """weights on the host (for the oracle) and the device (for the call)"""

    def __init__(self, M, Q, oracle, seed, E=512, FE=256, NE=16, NU=4, t_gu=100, t_d=100, FS=256, t_sgu=None,
                 t_sd=None, router=0, shexp=True, gate_vec=True):
        self.E, self.FE, self.NE, self.NU, self.FS = E, FE, NE, NU, FS if shexp else 0
        self.t_gu, self.t_d = t_gu, t_d
        self.t_sgu, self.t_sd = (t_gu if t_sgu is None else t_sgu), (t_d if t_sd is None else t_sd)
        g = lambda s, n, k: synth.gaussian(seed + s, n * k, 0, 0.05).reshape(n, k)
        self.gate = oracle.quantize(t_gu, g(1, NE * FE, E))
        self.up = oracle.quantize(t_gu, g(2, NE * FE, E))
        self.down = oracle.quantize(t_d, g(3, NE * E, FE))
        rw = g(4, NE, E)
        self.router_t = router
        if router == 0:
            self.router = rw.view(np.uint8)
        elif router == 30:
            u = rw.view(np.uint32)
            self.router = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8)
        else:
            self.router = oracle.quantize(router, rw)
        self.keep = [dev(self.gate), dev(self.up), dev(self.down), dev(self.router)]
        w = M.MoeWeights()
        w.n_embd, w.n_ff_exp, w.n_expert, w.n_expert_used = E, FE, NE, NU
        w.type_gate_up, w.type_down = t_gu, t_d
        w.gate_exps, w.up_exps, w.down_exps = [t.data_ptr() for t in self.keep[:3]]
        w.rb_gate_up, w.rb_down = self.gate.shape[1], self.down.shape[1]
        w.type_router, w.router, w.rb_router = router, self.keep[3].data_ptr(), self.router.size // NE
        self.shexp = shexp
        self.gvec = None
        if shexp:
            self.sgate = oracle.quantize(self.t_sgu, g(5, FS, E))
            self.sup = oracle.quantize(self.t_sgu, g(6, FS, E))
            self.sdown = oracle.quantize(self.t_sd, g(7, E, FS))
            sk = [dev(self.sgate), dev(self.sup), dev(self.sdown)]
            self.keep += sk
            w.n_ff_shexp = FS
            w.type_shexp_gate_up, w.type_shexp_down = self.t_sgu, self.t_sd
            w.gate_shexp, w.up_shexp, w.down_shexp = [t.data_ptr() for t in sk]
            w.rb_shexp_gate_up, w.rb_shexp_down = self.sgate.shape[1], self.sdown.shape[1]
            if gate_vec:
                self.gvec = synth.gaussian(seed + 8, E, 0, 0.05)
                gv = dev(self.gvec)
                self.keep.append(gv)
                w.shexp_gate = gv.data_ptr()
        self.w = w

    def logits(self, Q, x):
        """the router logits as the call computes them (the same launch)"""
        import torch
        T = x.shape[0]
        y = torch.empty((T, self.NE), dtype=torch.float32, device="cuda")
        L = Q.lib()
        if self.router_t in (0, 1, 30):
            xh = torch.empty(T * self.E, dtype=torch.uint16, device="cuda")
            assert L.qmatvec_launch_batch_h(self.router_t, p(self.keep[3]), self.w.rb_router, p(dev(x)), p(xh),
                                            T * self.E * 2, p(y), self.NE, self.E, T, None) == 0
        else:
            q = Q.Q8(((T * self.E + 255) // 256) * 256)
            Q.quantize(dev(x.reshape(-1)), T * self.E, q)
            Q.launch_q8_batch(self.router_t, self.keep[3], q, y, self.NE, self.NE, self.E, T)
        return host(y)

    def run(self, M, Q, x, keep_ws=False):
        import torch
        T = x.shape[0]
        q = Q.Q8(((T * self.E + 255) // 256) * 256)
        xd = dev(x)
        Q.quantize(xd.reshape(-1), T * self.E, q)
        nb = M.workspace_bytes(self.w, T)
        assert nb > 0
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        out = torch.full((T, self.E), float("nan"), dtype=torch.float32, device="cuda")
        M.ffn(self.w, xd, q, T, out, ws)
        return (host(out), host(ws)) if keep_ws else host(out)

    def check_stages(self, M, oracle, x, logits, out, ws):
        moe_stages.check(M, oracle, self.w, x, logits, out, ws, self.down, self.t_d, self.NU,
                         self.sdown if self.shexp else None, self.t_sd, self.FS)

    def oracle(self, oracle, x, logits):
        T, E, FE, NU = x.shape[0], self.E, self.FE, self.NU
        ids, wts = oracle.moe_router(logits, NU)
        rg, rd = self.gate.shape[1], self.down.shape[1]
        down = np.zeros((T, NU, E), np.float32)
        shared = np.zeros((T, E), np.float32) if self.shexp else None
        sg = None
        for t in range(T):
            a = oracle.quantize_act(x[t], self.t_gu in KQ)
            for j in range(NU):
                e = ids[t, j]
                gg = oracle.matvec(self.t_gu, self.gate[e * FE:(e + 1) * FE], FE, E, a, False)[0]
                uu = oracle.matvec(self.t_gu, self.up[e * FE:(e + 1) * FE], FE, E, a, False)[0]
                h = oracle.swiglu(gg, uu)
                down[t, j] = oracle.matvec(self.t_d, self.down[e * E:(e + 1) * E], E, FE,
                                           oracle.quantize_act(h, self.t_d in KQ), False)[0]
            if self.shexp:
                a2 = oracle.quantize_act(x[t], self.t_sgu in KQ)
                gg = oracle.matvec(self.t_sgu, self.sgate, self.FS, E, a2, False)[0]
                uu = oracle.matvec(self.t_sgu, self.sup, self.FS, E, a2, False)[0]
                shared[t] = oracle.matvec(self.t_sd, self.sdown, E, self.FS,
                                          oracle.quantize_act(oracle.swiglu(gg, uu), self.t_sd in KQ), False)[0]
        if self.gvec is not None:
            sg = np.array([oracle.shared_gate(x[t], self.gvec) for t in range(T)], np.float32)
        return oracle.moe_combine(down, wts, shared, sg), ids


def acts(seed, T, E):
    return synth.gaussian(seed, T * E).reshape(T, E)


def close(got, want):
    scale = np.abs(want).max(axis=1, keepdims=True) + 1e-30
    err = (np.abs(got - want) / scale).max()
    assert err <= 2e-3, f"max error {err:.3g} of the row maximum"


@pytest.mark.parametrize("t_gu,t_d,E,FE", [(100, 100, 512, 256), (12, 14, 512, 512), (101, 8, 512, 256)])
def test_slot_form_same_bits_as_plain_sequence(M, Q, oracle, t_gu, t_d, E, FE):
    """one token, a shared expert of the experts' shape: the 3-launch slot form equals the plain sequence (router,
    gate / up pair, shared gate / up, SwiGLUs with their quantization, down, shared down, combine) bit for bit"""
    import torch
    lay = Layer(M, Q, oracle, 100 + t_gu, E=E, FE=FE, t_gu=t_gu, t_d=t_d, FS=FE)
    assert M.lib().purhie_moe_shared_as_slot(C.byref(lay.w), 1) == 1
    x = acts(7, 1, E)
    got = lay.run(M, Q, x)
    # the plain sequence, launch by launch
    L, ML = Q.lib(), M.lib()
    NE, NU = lay.NE, lay.NU
    logits = dev(lay.logits(Q, x))
    xd = dev(x)
    q = Q.Q8(((E + 255) // 256) * 256)
    Q.quantize(xd.reshape(-1), E, q)
    ids = torch.zeros((1, NU), dtype=torch.int32, device="cuda")
    wts = torch.zeros((1, NU), dtype=torch.float32, device="cuda")
    sg = torch.zeros(1, dtype=torch.float32, device="cuda")
    gv = lay.keep[-1]
    assert ML.gpu_moe_router(p(logits), p(xd), p(gv), p(ids), p(wts), p(sg), NE, NU, E, 1, None, 0) == 0
    g = torch.zeros((NU, FE), device="cuda")
    u = torch.zeros((NU, FE), device="cuda")
    Q.launch_q8_id_x(t_gu, lay.keep[0], lay.keep[1], None, None, ids, NU, 0, q, g, u, FE, E, 1)
    sgt, sut = torch.zeros(FE, device="cuda"), torch.zeros(FE, device="cuda")
    Q.launch_q8_batch(t_gu, lay.keep[4], q, sgt, FE, FE, E, 1)
    Q.launch_q8_batch(t_gu, lay.keep[5], q, sut, FE, FE, E, 1)
    act = torch.zeros(NU * FE, device="cuda")
    qx = Q.Q8(((NU * FE + 255) // 256) * 256)
    assert ML.gpu_swiglu(p(g), p(u), p(act), NU * FE, qx.ref, None) == 0
    dn = torch.zeros((NU, E), device="cuda")
    Q.launch_q8_id_x(t_d, lay.keep[2], None, None, None, ids, NU, 1, qx, dn, None, E, FE, 1)
    sact = torch.zeros(FE, device="cuda")
    qs = Q.Q8(((FE + 255) // 256) * 256)
    assert ML.gpu_swiglu(p(sgt), p(sut), p(sact), FE, qs.ref, None) == 0
    sh = torch.zeros(E, device="cuda")
    Q.launch_q8_batch(t_d, lay.keep[6], qs, sh, E, E, FE, 1)
    out = torch.zeros((1, E), device="cuda")
    assert ML.gpu_moe_combine(p(dn), p(wts), p(sh), p(sg), p(out), NU, E, 1, None) == 0
    assert np.array_equal(got.view(np.uint32), host(out).view(np.uint32))


@pytest.mark.parametrize("T,t_gu,t_d,E,FE,NE,NU", [
    (1, 100, 100, 512, 256, 16, 4),
    (3, 101, 8, 512, 256, 16, 4),
    (7, 100, 100, 1024, 768, 32, 8),   # 13 row tiles of 85 in the down launch
    (1, 100, 100, 2048, 768, 12, 8),   # config 4's widths (hidden 2048, FFN 768, top-8)
    (2, 12, 14, 512, 512, 16, 4),      # a Q8_K down matvec: SwiGLU in its own launch
])
def test_routed_form_same_bits_as_plain_sequence(M, Q, oracle, T, t_gu, t_d, E, FE, NE, NU):
    """a few tokens, no shared expert: the routing inside the gate / up launch and, for a Q8_0-activation down
    type, SwiGLU inside the down launch give the plain sequence's bits (router, gate / up pair, SwiGLU with its
    quantization, down, combine). Two calls on one workspace: the second starts from what the first left."""
    import torch
    lay = Layer(M, Q, oracle, 600 + T, E=E, FE=FE, NE=NE, NU=NU, t_gu=t_gu, t_d=t_d, shexp=False)
    x = acts(70 + T, T, E)
    q = Q.Q8(((T * E + 255) // 256) * 256)
    xd = dev(x)
    Q.quantize(xd.reshape(-1), T * E, q)
    ws = torch.empty(M.workspace_bytes(lay.w, T), dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(2):
        out = torch.full((T, E), float("nan"), dtype=torch.float32, device="cuda")
        M.ffn(lay.w, xd, q, T, out, ws)
        outs.append(host(out))
    L, ML = Q.lib(), M.lib()
    logits = dev(lay.logits(Q, x))
    ids = torch.zeros((T, NU), dtype=torch.int32, device="cuda")
    wts = torch.zeros((T, NU), dtype=torch.float32, device="cuda")
    assert ML.gpu_moe_router(p(logits), None, None, p(ids), p(wts), None, NE, NU, E, T, None, 0) == 0
    g = torch.zeros((T * NU, FE), device="cuda")
    u = torch.zeros((T * NU, FE), device="cuda")
    Q.launch_q8_id_x(t_gu, lay.keep[0], lay.keep[1], None, None, ids, NU, 0, q, g, u, FE, E, T)
    act = torch.zeros(T * NU * FE, device="cuda")
    qx = Q.Q8(((T * NU * FE + 255) // 256) * 256)
    assert ML.gpu_swiglu(p(g), p(u), p(act), T * NU * FE, qx.ref, None) == 0
    dn = torch.zeros((T * NU, E), device="cuda")
    Q.launch_q8_id_x(t_d, lay.keep[2], None, None, None, ids, NU, 1, qx, dn, None, E, FE, T)
    want = torch.zeros((T, E), device="cuda")
    assert ML.gpu_moe_combine(p(dn), p(wts), None, None, p(want), NU, E, T, None) == 0
    want = host(want)
    for got in outs:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("case", [
    dict(T=1),                                                     # slot form
    dict(T=5),                                                     # per-token matvecs
    dict(T=24),                                                    # grouped GEMMs
    dict(T=3, shexp=False),                                        # routed experts only
    dict(T=12, t_gu=12, t_d=14, E=512, FE=512, FS=768, t_sgu=12, t_sd=14),  # K-quants, a wider shared expert
    dict(T=1, t_gu=12, t_d=13, E=512, FE=256, FS=512, t_sgu=12, t_sd=12),   # one token, no slot (other width)
    dict(T=40, router=30, gate_vec=False),                         # BF16 router through its GEMM, ungated shexp
    dict(T=9, router=8, t_gu=39, t_d=40),                          # Q8_0 router, MXFP4 / NVFP4 experts
])
def test_matches_oracle(M, Q, oracle, case):
    case = dict(case)
    T = case.pop("T")
    lay = Layer(M, Q, oracle, 300 + T, **case)
    x = acts(40 + T, T, lay.E)
    got, ws = lay.run(M, Q, x, keep_ws=True)
    logits = lay.logits(Q, x)
    lay.check_stages(M, oracle, x, logits, got, ws)
    # the whole layer against the oracle's own composition: a reading (a re-quantized SwiGLU value can move by a
    # step where the fp32 sums differ in order, so this bound is looser than the stages')
    want, _ = lay.oracle(oracle, x, logits)
    close(got, want)


def test_dispatch_rules(M, Q, oracle):
    L = M.lib()
    same = Layer(M, Q, oracle, 500)
    wider = Layer(M, Q, oracle, 501, FS=512)
    none = Layer(M, Q, oracle, 502, shexp=False)
    assert L.purhie_moe_shared_as_slot(C.byref(same.w), 1) == 1
    assert L.purhie_moe_shared_as_slot(C.byref(same.w), 2) == 0
    assert L.purhie_moe_shared_as_slot(C.byref(wider.w), 1) == 0
    assert L.purhie_moe_shared_as_slot(C.byref(none.w), 1) == 0
    # the grouped form needs the tile arrays, the slot form one more slot: the workspace sizes differ
    b1, b7, b8 = (M.workspace_bytes(same.w, T) for T in (1, 7, 8))
    assert 0 < b1 < b7 < b8
    bad = M.MoeWeights.from_buffer_copy(same.w)
    bad.n_expert_used = 64
    assert M.workspace_bytes(bad, 1) == 0
    bad = M.MoeWeights.from_buffer_copy(same.w)
    bad.rb_down += 1
    assert M.workspace_bytes(bad, 1) == 0
    bad = M.MoeWeights.from_buffer_copy(same.w)
    bad.n_embd = 500  # ROCmFP4 needs K % 64
    assert M.workspace_bytes(bad, 1) == 0
    import torch
    q = Q.Q8(512)
    x = torch.zeros(512, device="cuda")
    out = torch.zeros(512, device="cuda")
    ws = torch.empty(b1, dtype=torch.uint8, device="cuda")
    small = torch.empty(b1 - 256, dtype=torch.uint8, device="cuda")
    assert L.purhie_moe_ffn(C.byref(same.w), p(x), q.ref, 1, p(out), p(small), small.numel(), None) == 1
    assert L.purhie_moe_ffn(C.byref(same.w), p(x), q.ref, 2, p(out), p(ws), ws.numel(), None) == 1  # q8 too small
    assert L.purhie_moe_ffn(C.byref(same.w), p(x), q.ref, 1, p(out), C.c_void_p(ws.data_ptr() + 16), b1 - 16,
                            None) == 1  # workspace not 256-byte aligned
