"""Output scales (qmatvec_set_out_scale / qmatvec_drop_out_scales; reference src/qmatvec.h:21-26,
src/qmatvec.cpp:175-253): NVFP4's global scale per matrix or per stacked expert. With a scale registered, every
launch on the matrix returns its unscaled outputs times the scale, rounded once: the decode kernels (tile and
per-wave, 1 and 3 tokens), the prefill GEMMs, the expert-indexed matvec (per-expert scales, and the extra matrix's
own scale for an id of -1) and the expert-tiled GEMM. Dropping the owner's registrations restores the unscaled
outputs bit for bit."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    yield qmatvec
    qmatvec.lib().qmatvec_set_prefill(0)


@pytest.fixture(params=["tile", "wave"])
def kpath(request, monkeypatch):
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


def pinned(vals):
    """scale values readable by the host and the GPU for as long as they are registered"""
    import torch
    return torch.tensor(vals, dtype=torch.float32).pin_memory()


def p(t):
    return C.c_void_p(t.data_ptr())


def scaled(v, s):
    return (np.asarray(v, np.float32) * np.float32(s)).astype(np.float32)


def batch(Q, t, Wd, x, N, K):
    import torch
    T = x.shape[0]
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    y = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
    Q.launch_q8_batch(t, Wd, q, y, N, N, K, T)
    return host(y)


@pytest.mark.parametrize("t", (40, 100, 12))
def test_dense_scale(Q, oracle, kpath, t):
    N, K = 512, 1024
    L = Q.lib()
    W = oracle.quantize(t, synth.gaussian(21 + t, N * K, 0, 0.02).reshape(N, K))
    Wd = dev(W)
    owner = C.c_void_p(0x5CA1E)
    s = pinned([0.37])
    for T, prefill in ((1, 0), (3, 0), (70, 1)):
        L.qmatvec_set_prefill(prefill)
        x = synth.gaussian(30 + T, T * K).reshape(T, K)
        base = batch(Q, t, Wd, x, N, K)
        assert L.qmatvec_set_out_scale(owner, p(Wd), Wd.numel(), p(s), 1) == 0
        try:
            got = batch(Q, t, Wd, x, N, K)
        finally:
            L.qmatvec_drop_out_scales(owner)
        assert np.array_equal(got.view(np.uint32), scaled(base, 0.37).view(np.uint32)), (T, prefill)
        assert np.array_equal(batch(Q, t, Wd, x, N, K).view(np.uint32), base.view(np.uint32))
    L.qmatvec_set_prefill(0)
    # a registration elsewhere leaves this matrix alone; a bad count is refused
    other = dev(np.zeros(4096, np.uint8))
    assert L.qmatvec_set_out_scale(owner, p(other), other.numel(), p(s), 1) == 0
    x = synth.gaussian(40, K).reshape(1, K)
    try:
        assert np.array_equal(batch(Q, t, Wd, x, N, K).view(np.uint32), batch(Q, t, Wd, x, N, K).view(np.uint32))
        assert L.qmatvec_set_out_scale(owner, p(other), 4095, p(s), 2) == -1
    finally:
        L.qmatvec_drop_out_scales(owner)


@pytest.mark.parametrize("t", (40, 12))
def test_expert_scales(Q, oracle, kpath, t):
    """stacked experts registered with one scale each (n = E); the extra matrix (id -1) with its own"""
    import torch
    E, N, K, n_used, T = 4, 256, 1024, 3, 2
    L = Q.lib()
    W = oracle.quantize(t, synth.gaussian(50 + t, E * N * K, 0, 0.02).reshape(E * N, K))
    Wx = oracle.quantize(t, synth.gaussian(51 + t, N * K, 0, 0.02).reshape(N, K))
    Wd, Wxd = dev(W), dev(Wx)
    ids = np.array([[3, 0, -1], [1, 3, 2]], dtype=np.int32)
    x = synth.gaussian(52, T * K).reshape(T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)

    def run():
        y = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
        Q.launch_q8_id_x(t, Wd, None, Wxd, None, dev(ids), n_used, 0, q, y, None, N, K, T)
        return host(y)

    es = [0.5, 1.75, 0.0625, 3.0]
    s, sx = pinned(es), pinned([0.8125])
    owner = C.c_void_p(0xE5)
    base = run()
    assert L.qmatvec_set_out_scale(owner, p(Wd), Wd.numel(), p(s), E) == 0
    assert L.qmatvec_set_out_scale(owner, p(Wxd), Wxd.numel(), p(sx), 1) == 0
    try:
        got = run()
    finally:
        L.qmatvec_drop_out_scales(owner)
    for tt in range(T):
        for j in range(n_used):
            e = ids[tt, j]
            f = 0.8125 if e < 0 else es[e]
            r = tt * n_used + j
            assert np.array_equal(got[r].view(np.uint32), scaled(base[r], f).view(np.uint32)), (tt, j, e)
    assert np.array_equal(run().view(np.uint32), base.view(np.uint32))


@pytest.mark.parametrize("t", (40, 100, 39))
def test_expert_tiled_gemm_scales(Q, oracle, t):
    """the expert-tiled GEMM (grouped prefill) applies expert tile_e[k]'s scale to every entry of tile k"""
    import torch
    E, N, K, n_used, T = 8, 256, 1024, 4, 40
    L = Q.lib()
    W = oracle.quantize(t, synth.gaussian(60 + t, E * N * K, 0, 0.02).reshape(E * N, K))
    Wd = dev(W)
    ids = (synth.splitmix64(61, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    tile = L.qmatvec_id_batch_tile(t, N, K)
    g = oracle.moe_group(ids, E, tile)
    x = synth.gaussian(62, T * K).reshape(T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    bufs = [dev(np.array([g["n_tiles"]], np.int32)), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]),
            dev(g["tok_rows"]), dev(g["pair_rows"])]

    def run():
        y = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
        rc = L.qmatvec_launch_q8_id_batch(t, p(Wd), Q.row_size(t, K), q.ref, p(y), N, K, g["n_tiles"], tile,
                                          *[p(b) for b in bufs], None)
        assert rc == 0
        return host(y)

    es = [0.25 * (e + 1) for e in range(E)]
    s = pinned(es)
    owner = C.c_void_p(0x7E)
    base = run()
    assert L.qmatvec_set_out_scale(owner, p(Wd), Wd.numel(), p(s), E) == 0
    try:
        got = run()
    finally:
        L.qmatvec_drop_out_scales(owner)
    for tt in range(T):
        for j in range(n_used):
            r = tt * n_used + j
            f = es[ids[tt, j]]
            assert np.array_equal(got[r].view(np.uint32), scaled(base[r], f).view(np.uint32)), (tt, j)
