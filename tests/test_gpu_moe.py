"""GPU parity of the MoE glue (include/moe_ops.h) against the oracle's restatement of src/gpu_ops.hip:103-330:
router selection exact, weights and the shared gate to float tolerance, combine bit for bit (both sides round
every product and sum), grouping counts / tiles exact with every expert run holding exactly its entries, and
the fused SwiGLU quantization bit-identical to quantizing the SwiGLU output on its own."""
import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    from purhie_amd import moe
    moe.lib()
    return moe


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("T,E,n_used", [(1, 128, 8), (512, 128, 8), (7, 256, 8), (3, 1024, 64), (5, 16, 4),
                                        (4, 64, 8), (6, 65, 8), (3, 100, 6), (4, 127, 16), (3, 129, 8),
                                        (300, 256, 8), (4, 256, 16), (4, 256, 17), (5, 192, 1), (3, 255, 12)])
def test_router(M, oracle, T, E, n_used):
    import torch
    logits = synth.gaussian(900 + T + E, T * E).reshape(T, E)
    if T >= 3:
        logits[1, 5] = logits[1, 9] = logits[1].max() + 1.0  # equal leaders: the lower expert first
        logits[2, :] = 0.25                                    # all equal
    ids = torch.full((T, n_used), -9, dtype=torch.int32, device="cuda")
    wts = torch.zeros((T, n_used), dtype=torch.float32, device="cuda")
    M.router(dev(logits), ids, wts, E, n_used, T)
    want_ids, want_w = oracle.moe_router(logits, n_used)
    assert np.array_equal(host(ids), want_ids)
    assert np.allclose(host(wts), want_w, rtol=2e-6, atol=1e-8)


@pytest.mark.parametrize("E", [128, 256, 200])
def test_router_shared_gate_and_stride(M, oracle, E):
    import torch
    T, n_used, n = 6, 8, 2048
    logits = synth.gaussian(950, T * E).reshape(T, E)
    x = synth.gaussian(951, T * n).reshape(T, n)
    w = synth.gaussian(952, n, 0, 0.02)
    ids = torch.full((T, n_used + 1), -9, dtype=torch.int32, device="cuda")
    wts = torch.zeros((T, n_used), dtype=torch.float32, device="cuda")
    sg = torch.zeros(T, dtype=torch.float32, device="cuda")
    M.router(dev(logits), ids, wts, E, n_used, T, x=dev(x), w_shexp=dev(w), sg=sg, n=n, ids_stride=n_used + 1)
    got = host(ids)
    want_ids, _ = oracle.moe_router(logits, n_used)
    assert np.array_equal(got[:, :n_used], want_ids)
    assert np.all(got[:, n_used] == -1)
    want_sg = np.array([oracle.shared_gate(x[t], w) for t in range(T)], np.float32)
    assert np.allclose(host(sg), want_sg, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("variant", ["plain", "shared_gated", "shared", "scaled", "unit_weights"])
def test_combine_bit_exact(M, oracle, variant):
    import torch
    T, J, n, E = 5, 8, 2048, 128
    down = synth.gaussian(960, T * J * n).reshape(T, J, n)
    w = np.abs(synth.gaussian(961, T * J)).reshape(T, J)
    sh = synth.gaussian(962, T * n).reshape(T, n)
    sg = np.abs(synth.gaussian(963, T))
    ids = (synth.splitmix64(964, T * J) % np.uint64(E)).astype(np.int32).reshape(T, J)
    es = synth.gaussian(965, E)
    a = dict(plain=(w, None, None, None), shared_gated=(w, sh, sg, None), shared=(w, sh, None, None),
             scaled=(w, None, None, es), unit_weights=(None, sh, None, None))[variant]
    wts, shared, gate, scale = a
    out = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
    opt = lambda v: None if v is None else dev(v)
    M.combine(dev(down), opt(wts), out, J, n, T, shared=opt(shared), sg=opt(gate),
              ids=dev(ids) if scale is not None else None, exp_scale=opt(scale))
    want = oracle.moe_combine(down, wts, shared, gate, ids if scale is not None else None, scale)
    assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("T,n_used,E,tile", [(512, 8, 128, 64), (1999, 8, 160, 64), (1, 8, 128, 16), (37, 4, 16, 5),
                                             (0, 8, 128, 64)])
def test_group(M, oracle, T, n_used, E, tile):
    ids = (synth.splitmix64(970 + T, max(T, 1) * n_used) % np.uint64(E)).astype(np.int32)[:T * n_used]
    if T >= 37:
        ids[: 3 * n_used] = 3  # a heavy expert
    got = M.group(dev(ids if T else np.zeros(1, np.int32)), T, n_used, E, tile)
    if T == 0:
        assert got["n_tiles"] == 0
        return
    want = oracle.moe_group(ids.reshape(T, n_used), E, tile)
    assert got["n_tiles"] == want["n_tiles"] <= M.max_tiles(T, n_used, E, tile)
    for k in ("tile_e", "tile_start", "tile_n"):
        assert np.array_equal(got[k], want[k][:want["n_tiles"]]), k
    for k in range(got["n_tiles"]):
        s, n = got["tile_start"][k], got["tile_n"][k]
        assert np.all(ids[got["pair_rows"][s:s + n]] == got["tile_e"][k])
    # every expert's run holds exactly its entries (the order inside a run is free)
    cnt = np.bincount(ids, minlength=E)
    off = np.concatenate([[0], np.cumsum(cnt)])
    for e in range(E):
        run = np.sort(got["pair_rows"][off[e]:off[e + 1]])
        assert np.array_equal(run, np.nonzero(ids == e)[0])
    assert np.array_equal(got["tok_rows"], got["pair_rows"] // n_used)


@pytest.mark.parametrize("n", [768, 2048, 4096, 96, 4096 * 256, 4097 * 256 - 160, 100])
def test_swiglu_fused_quantize(M, oracle, n):
    """gpu_swiglu with both activation formats against the oracle; n from one block to past 4096 blocks (the
    wave-per-block kernel, four blocks a wave, with a ragged last block); n = 100 (n % 32 != 0) is the
    workgroup-per-block kernel's, with its Q8_0 refused"""
    import torch
    from purhie_amd import qmatvec as Q
    g = synth.gaussian(980 + n, n) * 3.0
    u = synth.gaussian(981 + n, n)
    out = torch.zeros(n, dtype=torch.float32, device="cuda")
    q = Q.Q8(((n + 255) // 256) * 256)
    if n % 32:
        with pytest.raises(Q.HipError):
            M.swiglu(dev(g), dev(u), out, n, q)
        with pytest.raises(Q.HipError):  # out NULL needs q8
            M.swiglu(dev(g), dev(u), None, n)
        M.swiglu(dev(g), dev(u), out, n)
        assert np.allclose(host(out), oracle.swiglu(g, u), rtol=1e-6, atol=1e-30)
        return
    M.swiglu(dev(g), dev(u), out, n, q)
    got = host(out)
    assert np.allclose(got, oracle.swiglu(g, u), rtol=1e-6, atol=1e-30)
    v = {k: host(t) for k, t in q.views(n).items()}
    a0 = oracle.quantize_act(got, kq=False)
    assert np.array_equal(v["q0"], a0["q"])
    assert np.array_equal(v["d0"].view(np.uint32), a0["d"].view(np.uint32))
    assert np.array_equal(v["s0"], a0["s0"])
    if n % 256 == 0:
        aK = oracle.quantize_act(got, kq=True)
        assert np.array_equal(v["qK"], aK["q"])
        assert np.array_equal(v["dK"].view(np.uint32), aK["d"].view(np.uint32))
        assert np.array_equal(v["bsK"], aK["bs"])
    out2 = torch.zeros(n, dtype=torch.float32, device="cuda")
    M.swiglu(dev(g), dev(u), out2, n)  # without quantization: the same values
    assert np.array_equal(host(out2).view(np.uint32), got.view(np.uint32))
    # buffers one float off 16-byte alignment go to the workgroup-per-block kernel: the same bits
    gb, ub = torch.zeros(n + 1, dtype=torch.float32, device="cuda"), torch.zeros(n + 1, dtype=torch.float32, device="cuda")
    gb[1:] = dev(g)
    ub[1:] = dev(u)
    out3 = torch.zeros(n + 1, dtype=torch.float32, device="cuda")
    q3 = Q.Q8(((n + 255) // 256) * 256)
    M.swiglu(gb[1:], ub[1:], out3[1:], n, q3)
    assert np.array_equal(host(out3[1:]).view(np.uint32), got.view(np.uint32))
    v3 = {k: host(t) for k, t in q3.views(n).items()}
    for k in v:
        assert np.array_equal(v3[k].view(np.uint8), v[k].view(np.uint8)), k
    # out NULL with q8 (the MoE layer's call): only the quantized form, the same bits, from both kernels
    for gg, uu in ((dev(g), dev(u)), (gb[1:], ub[1:])):
        q4 = Q.Q8(((n + 255) // 256) * 256)
        M.swiglu(gg, uu, None, n, q4)
        v4 = {k: host(t) for k, t in q4.views(n).items()}
        for k in v:
            assert np.array_equal(v4[k].view(np.uint8), v[k].view(np.uint8)), k


@pytest.mark.parametrize("n,T", [(2560, 1), (5120, 3), (2048, 16), (1024, 40), (9728, 9)])
def test_add_rmsnorm_fused_quantize(M, oracle, n, T):
    """gpu_add_rmsnorm (src/gpu_ops.hip:17-100): x_out = x_in + add bit for bit (one fp32 add), y within a few
    ulps of the float64 RMSNorm of it, the fused quantization bit-identical to the oracle's quantizer on the y it
    wrote (both formats), and each row the same bits as that row normalized alone (the one-row kernel against
    the many-rows one)"""
    import torch
    from purhie_amd import qmatvec as Q
    eps = 1e-6
    x = synth.gaussian(990 + n + T, T * n).reshape(T, n)
    a = synth.gaussian(991 + n + T, T * n).reshape(T, n) * np.float32(0.5)
    w = (synth.gaussian(992 + n, n) * np.float32(0.1) + np.float32(1.0)).astype(np.float32)
    y = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
    xo = torch.full((T, n), float("nan"), dtype=torch.float32, device="cuda")
    q = Q.Q8(T * n)
    M.add_rmsnorm(dev(x), y, n, T, eps, add=dev(a), x_out=xo, w=dev(w), q8=q)
    s = x + a
    assert np.array_equal(host(xo).view(np.uint32), s.view(np.uint32))
    got = host(y)
    s64 = s.astype(np.float64)
    want = s64 / np.sqrt((s64 * s64).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)
    assert np.all(np.abs(got - want) <= 4e-7 * np.abs(want) + 1e-30), np.abs((got - want) / want).max()
    v = {k: host(t) for k, t in q.views(T * n).items()}
    a0, aK = oracle.quantize_act(got, kq=False), oracle.quantize_act(got, kq=True)
    assert np.array_equal(v["q0"], a0["q"]) and np.array_equal(v["d0"].view(np.uint32), a0["d"].view(np.uint32))
    assert np.array_equal(v["s0"], a0["s0"])
    assert np.array_equal(v["qK"], aK["q"]) and np.array_equal(v["dK"].view(np.uint32), aK["d"].view(np.uint32))
    assert np.array_equal(v["bsK"], aK["bs"])
    for r in range(min(T, 3)):
        y1 = torch.zeros(n, dtype=torch.float32, device="cuda")
        x1 = torch.zeros(n, dtype=torch.float32, device="cuda")
        M.add_rmsnorm(dev(x[r]), y1, n, 1, eps, add=dev(a[r]), x_out=x1, w=dev(w))
        assert np.array_equal(host(y1).view(np.uint32), got[r].view(np.uint32)), r
    # without add (x_out untouched) and without gamma
    y2 = torch.zeros((T, n), dtype=torch.float32, device="cuda")
    xo2 = torch.full((T, n), 7.0, dtype=torch.float32, device="cuda")
    M.add_rmsnorm(dev(s), y2, n, T, eps, x_out=xo2)
    want2 = s64 / np.sqrt((s64 * s64).mean(axis=1, keepdims=True) + eps)
    assert np.all(np.abs(host(y2) - want2) <= 4e-7 * np.abs(want2) + 1e-30)
    assert np.all(host(xo2) == 7.0)


def test_add_rmsnorm_bad_arguments(M):
    import torch
    from purhie_amd import qmatvec as Q
    L = M.lib()
    x = torch.zeros(512, device="cuda")
    q = Q.Q8(256)
    p = lambda t: __import__("ctypes").c_void_p(t.data_ptr())
    assert L.gpu_add_rmsnorm(p(x), p(x), p(x), None, p(x), 256, 1, 1e-6, None, None) == 1  # x_out aliases x_in
    assert L.gpu_add_rmsnorm(p(x), None, None, None, p(x), 200, 1, 1e-6, q.ref, None) == 1  # n % 256
    assert L.gpu_add_rmsnorm(p(x), None, None, None, p(x), 256, 2, 1e-6, q.ref, None) == 1  # T n > max_k


@pytest.mark.parametrize("kpath", ["tile", "wave"])
@pytest.mark.parametrize("t,T,E,n_used,N,K", [(100, 1, 128, 8, 768, 2048), (12, 1, 128, 8, 768, 2048),
                                              (100, 3, 256, 8, 512, 1024), (40, 2, 64, 4, 256, 1024),
                                              (100, 1, 300, 8, 256, 1024), (100, 2, 100, 6, 256, 1024),
                                              (8, 1, 16, 4, 64, 16384), (8, 1, 16, 4, 64, 24576),
                                              (8, 1, 16, 4, 64, 32768)])
def test_routed_pair_same_bits(M, oracle, kpath, t, T, E, n_used, N, K):
    """qmatvec_launch_q8_id_pair_routed (routing inside the gate / up pair launch) gives gpu_moe_router's ids and
    weights and qmatvec_launch_q8_id_pair's outputs bit for bit: on the tile kernel (n_expert <= 256) and through
    the two launches it falls back to (n_expert 300, the per-wave path, and a K whose tile's LDS
    would pass 64 KiB: Q8_0 at K = 32768; at K = 24576 the tile and the router's LDS within it take 62.5 KiB)"""
    import ctypes as C
    import torch
    from purhie_amd import qmatvec as Q
    prev = Q.decode_path(1 if kpath == "tile" else 0)
    try:
        W = torch.empty((E * N, Q.row_size(t, K)), dtype=torch.uint8, device="cuda")
        W2 = torch.empty_like(W)
        for i, w in enumerate((W, W2)):
            src = synth.gaussian_torch(torch, E * 31 + K + i, E * N * K, 0.0, 0.02).reshape(E * N, K)
            Q.encode_device(t, src, w, E * N, K)
        logits = synth.gaussian(950 + E, T * E).reshape(T, E)
        if T >= 2:
            logits[1, 3] = logits[1, 7] = logits[1].max() + 0.5  # equal leaders
        lg = dev(logits)
        x = dev(synth.gaussian(951, T * K))
        q = Q.Q8(((T * K + 255) // 256) * 256)
        Q.quantize(x, T * K, q)
        p = lambda a: C.c_void_p(a.data_ptr())
        L = Q.lib()
        outs = []
        for routed in (False, True):
            ids = torch.full((T, n_used), -9, dtype=torch.int32, device="cuda")
            wts = torch.full((T, n_used), float("nan"), device="cuda")
            y = torch.full((T * n_used, N), float("nan"), device="cuda")
            y2 = torch.full((T * n_used, N), float("nan"), device="cuda")
            rb = Q.row_size(t, K)
            if routed:
                assert L.qmatvec_launch_q8_id_pair_routed(t, p(W), p(W2), rb, p(lg), E, p(ids), p(wts), n_used, q.ref,
                                                          p(y), p(y2), N, K, T, None) == 0
            else:
                M.router(lg, ids, wts, E, n_used, T)
                assert L.qmatvec_launch_q8_id_pair(t, p(W), p(W2), rb, p(ids), n_used, 0, q.ref, p(y), p(y2), N, K, T,
                                                   None) == 0
            outs.append([host(a) for a in (ids, wts, y, y2)])
        for a, b in zip(*outs):
            assert np.isfinite(a.astype(np.float64)).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        Q.decode_path(prev)
