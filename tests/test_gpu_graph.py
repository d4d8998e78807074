"""The launch paths allocate nothing: config 3's ROCmFP4 prefill GEMM (qmatvec_launch_q8_batch), a 24-token MoE
FFN at config 4's sizes (purhie_moe_ffn: ROCmFP4 experts, and the mixed Q4_K gate / up, Q6_K down form), and the
float-activation, LM-head, low-rank and SwiGLU entries are captured into a HIP graph whose nodes are all kernel launches (no memory alloc / free, memset or copy nodes), and
every replay of the graph, with eager work and synchronisations between replays, gives the eager call's bits."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu

NODE_KERNEL = 0  # hipGraphNodeTypeKernel (hipGraphNodeTypeMemAlloc = 10, hipGraphNodeTypeMemFree = 11)
CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal: a synchronous allocation in this thread fails the capture


@pytest.fixture(scope="module")
def hip():
    import torch
    torch.cuda.init()
    h = C.CDLL("libamdhip64.so.7")  # the runtime the process already holds (torch's, and the library's)
    for f in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphGetNodes", "hipGraphNodeGetType",
              "hipGraphInstantiate", "hipGraphLaunch", "hipGraphExecDestroy", "hipGraphDestroy",
              "hipStreamSynchronize"):
        getattr(h, f).restype = C.c_int
    return h


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
    """N x K ~N(0, 0.02) weights encoded as type t by the library's GPU encoder"""
    import torch
    src = synth.gaussian_torch(torch, seed, N * K, 0.0, 0.02).reshape(N, K)
    out = torch.empty((N, Q.row_size(t, K)), dtype=torch.uint8, device="cuda")
    Q.encode_device(t, src, out, N, K)
    return out


class Captured:
    """the calls fn(stream) makes, captured on a fresh stream of default priority"""

    def __init__(self, hip, fn):
        import torch
        self.hip = hip
        self.s = torch.cuda.Stream()
        torch.cuda.synchronize()
        hs = C.c_void_p(self.s.cuda_stream)
        assert hip.hipStreamBeginCapture(hs, CAPTURE_THREAD_LOCAL) == 0
        try:
            fn(hs)
        finally:
            self.graph = C.c_void_p()
            rc = hip.hipStreamEndCapture(hs, C.byref(self.graph))
        assert rc == 0, f"hipStreamEndCapture: {rc} (a call in the capture was refused)"
        n = C.c_size_t(0)
        assert hip.hipGraphGetNodes(self.graph, None, C.byref(n)) == 0
        nodes = (C.c_void_p * n.value)()
        assert hip.hipGraphGetNodes(self.graph, nodes, C.byref(n)) == 0
        self.types = []
        for i in range(n.value):
            t = C.c_int(-1)
            assert hip.hipGraphNodeGetType(C.c_void_p(nodes[i]), C.byref(t)) == 0
            self.types.append(t.value)
        self.exe = C.c_void_p()
        assert hip.hipGraphInstantiate(C.byref(self.exe), self.graph, None, None, 0) == 0

    def replay(self):
        hs = C.c_void_p(self.s.cuda_stream)
        assert self.hip.hipGraphLaunch(self.exe, hs) == 0
        assert self.hip.hipStreamSynchronize(hs) == 0

    def close(self):
        self.hip.hipGraphExecDestroy(self.exe)
        self.hip.hipGraphDestroy(self.graph)


def replays_match(G, out, want, eager):
    """three replays, each after the output is overwritten by other work, give the eager bits"""
    import torch
    try:
        assert G.types and all(t == NODE_KERNEL for t in G.types), f"graph node types {sorted(set(G.types))}"
        for r in range(3):
            out.fill_(float("nan"))
            eager()  # the program's own eager work between replays
            torch.cuda.synchronize()
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            G.replay()
            got = out.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {r} differs from the eager call"
    finally:
        G.close()


def test_config3_gemm_graph(hip, Q):
    """config 3: ROCmFP4 W 17408 x 5120 over 2427 tokens (the prompt quantized inside the graph too)"""
    import torch
    t, N, K, T = 100, 17408, 5120, 2427
    W = encoded(Q, t, N, K, 3)
    x = dev(synth.with_outliers(synth.gaussian(4, T * K), 5, 0.001, 20.0))
    q = Q.Q8(((T * K + 255) // 256) * 256)
    y = torch.empty((T, N), dtype=torch.float32, device="cuda")

    def calls(stream=None):
        Q.quantize(x, T * K, q, stream)
        Q.launch_q8_batch(t, W, q, y, N, N, K, T, stream)

    calls()
    want = y.cpu().numpy()
    assert np.isfinite(want).all()
    G = Captured(hip, calls)
    replays_match(G, y, want, lambda: Q.launch_q8_batch(t, W, q, y, N, N, K, T))


@pytest.mark.parametrize("t_gu,t_d", [(100, 100), (12, 14)], ids=["rocmfp4", "q4k_q6k"])
def test_config4_moe_ffn_graph(hip, Q, M, t_gu, t_d):
    """config 4's sizes (hidden 2048, 128 experts of FFN 768, top 8), 24 tokens: the expert-grouped GEMM form"""
    import torch
    E, FE, NE, NU, T = 2048, 768, 128, 8, 24
    keep = [encoded(Q, t_gu, NE * FE, E, 11), encoded(Q, t_gu, NE * FE, E, 12), encoded(Q, t_d, NE * E, FE, 13),
            dev(synth.gaussian(14, NE * E, 0, 0.05))]
    w = M.MoeWeights()
    w.n_embd, w.n_ff_exp, w.n_expert, w.n_expert_used = E, FE, NE, NU
    w.type_gate_up, w.type_down = t_gu, t_d
    w.gate_exps, w.up_exps, w.down_exps = [k.data_ptr() for k in keep[:3]]
    w.rb_gate_up, w.rb_down = Q.row_size(t_gu, E), Q.row_size(t_d, FE)
    w.type_router, w.router, w.rb_router = 0, keep[3].data_ptr(), E * 4
    xd = dev(synth.gaussian(15, T * E).reshape(T, E))
    q = Q.Q8(((T * E + 255) // 256) * 256)
    nb = M.workspace_bytes(w, T)
    assert nb > 0
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    out = torch.empty((T, E), dtype=torch.float32, device="cuda")

    def calls(stream=None):
        Q.quantize(xd.reshape(-1), T * E, q, stream)
        M.ffn(w, xd, q, T, out, ws, stream)

    calls()
    want = out.cpu().numpy()
    assert np.isfinite(want).all() and np.abs(want).max() > 0
    G = Captured(hip, calls)
    replays_match(G, out, want, lambda: M.ffn(w, xd, q, T, out, ws))


def test_decode_side_entries_graph(hip, Q, M):
    """the float-activation matvec and batch over Q4_K (qmatvec_launch, _batch), the expert-indexed float matvec
    (qmatvec_launch_id), the split-Q8_0 LM head (qmatvec_quantize_rows_q8_0, qmatvec_launch_q8_0s), the low-rank
    matvec (qmatvec_launch_q8_lr) and gpu_swiglu with its quantizer, in one graph of kernel nodes whose replays give
    the eager bits"""
    import torch
    L = Q.lib()
    p = lambda t: C.c_void_p(t.data_ptr())
    N, K, T, E, NU = 1024, 2048, 3, 4, 2
    Wq = encoded(Q, 12, N, K, 21)
    We = encoded(Q, 12, E * N, K, 22)
    Wf = (synth.gaussian_torch(torch, 23, N * K, 0.0, 0.02).reshape(N, K)).to(torch.bfloat16).view(torch.uint8)
    Wl = encoded(Q, 101, N, 384, 24)
    x = dev(synth.gaussian(25, T * K).reshape(T, K))
    ids = dev(np.array([[1, 3], [0, 0], [2, -1]], np.int32))
    lo = dev(synth.gaussian(26, 320))
    g = dev(synth.gaussian(27, 8 * 256) * 3.0)
    u = dev(synth.gaussian(28, 8 * 256))
    q = Q.Q8(K)
    Q.quantize(x[0], K, q)
    qs = torch.empty(N * K, dtype=torch.int8, device="cuda")
    d = torch.empty(N * K // 32, dtype=torch.int16, device="cuda")
    qa = Q.Q8(8 * 256)
    outs = [torch.empty(N, device="cuda"), torch.empty((T, N), device="cuda"), torch.empty((T * NU, N), device="cuda"),
            torch.empty(N, device="cuda"), torch.empty(N, device="cuda"), torch.empty(8 * 256, device="cuda")]
    for o in outs:
        o.fill_(float("nan"))  # (the id -1 slot's row is never written)

    def calls(stream=None):
        assert L.qmatvec_launch(12, p(Wq), Wq.shape[1], p(x), p(outs[0]), N, K, stream) == 0
        assert L.qmatvec_launch_batch(12, p(Wq), Wq.shape[1], p(x), p(outs[1]), N, K, T, stream) == 0
        assert L.qmatvec_launch_id(12, p(We), We.shape[1], p(ids), NU, 0, p(x), p(outs[2]), N, K, T, stream) == 0
        assert L.qmatvec_quantize_rows_q8_0(30, p(Wf), 2 * K, N, K, p(qs), p(d), stream) == 0
        assert L.qmatvec_launch_q8_0s(p(qs), p(d), q.ref, p(outs[3]), N, K, stream) == 0
        assert L.qmatvec_launch_q8_lr(101, p(Wl), Wl.shape[1], p(lo), 320, 384, C.c_float(0.5), p(outs[4]), N,
                                      stream) == 0
        M.swiglu(g, u, outs[5], 8 * 256, qa, stream)

    def snapshot():
        torch.cuda.synchronize()
        return [o.cpu().numpy().copy() for o in outs] + [qa.mem.cpu().numpy().copy()]

    calls()
    want = snapshot()
    assert all(np.isfinite(want[i]).all() for i in (0, 1, 3, 4, 5))
    assert np.isfinite(np.delete(want[2], 2 * NU + 1, axis=0)).all() and np.isnan(want[2][2 * NU + 1]).all()
    G = Captured(hip, calls)
    try:
        assert G.types and all(t == NODE_KERNEL for t in G.types), f"graph node types {sorted(set(G.types))}"
        for r in range(3):
            for o in outs:
                o.fill_(float("nan"))
            qa.mem.fill_(0x55)
            calls()  # the program's own eager work between replays
            torch.cuda.synchronize()
            for o in outs:
                o.fill_(float("nan"))
            qa.mem.fill_(0x55)
            torch.cuda.synchronize()
            G.replay()
            got = snapshot()
            for i, (a, b) in enumerate(zip(got, want)):
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"replay {r}, output {i}"
    finally:
        G.close()
