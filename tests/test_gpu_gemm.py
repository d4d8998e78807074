"""GPU parity of the prefill GEMM (qmatvec_launch_q8_batch on the MFMA path) and of the MoE expert-tiled
GEMM (qmatvec_launch_q8_id_batch): every output within 1e-5 of sum |w x| of the oracle's per-token matvec
(the reference's tolerance for its WMMA path, tests/matvec_verify.cpp:230,272), and a token's result
independent of the batch it is computed in (split invariance, the reference's prefill-mode contract)."""
import numpy as np
import pytest

from purhie_amd import synth
from tests import parity

pytestmark = pytest.mark.gpu
TOL = 1e-5
GEMM_TYPES = (100, 101, 8, 12, 13, 14, 23, 39, 40)


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    yield qmatvec
    qmatvec.lib().qmatvec_set_prefill(0)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def acts(seed, T, K, outliers=True):
    x = synth.gaussian(seed, T * K)
    if outliers:  # config 3's 0.1% outliers x20
        x = synth.with_outliers(x, seed + 1, 0.001, 20.0)
    return x.reshape(T, K)


def run_batch(Q, t, Wd, x, N, K, ldy=None):
    import torch
    T = x.shape[0]
    ldy = ldy or N
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    y = torch.full((T, ldy), float("nan"), dtype=torch.float32, device="cuda")
    Q.launch_q8_batch(t, Wd, q, y, ldy, N, K, T)
    return host(y)[:, :N]


def check_tokens(oracle, t, W, N, K, x, got, what="prefill GEMM"):
    from purhie_amd import qmatvec
    for i in range(x.shape[0]):
        a = oracle.quantize_act(x[i], t in (12, 13, 14, 23))
        want, ref, mag = oracle.matvec(t, W, N, K, a)
        parity.check(f"{what} {qmatvec.NAMES[t]}", got[i], want, mag, ref, TOL)


@pytest.mark.parametrize("t", GEMM_TYPES)
@pytest.mark.parametrize("N,K,T", [(256, 1024, 70), (200, 2048, 130), (128, 5120, 33), (1024, 2048, 256)])
def test_gemm_parity(Q, oracle, t, N, K, T):
    W = oracle.quantize(t, synth.gaussian(N * 7 + K, N * K, 0, 0.02).reshape(N, K))
    x = acts(T + K, T, K)
    got = run_batch(Q, t, dev(W), x, N, K)
    check_tokens(oracle, t, W, N, K, x, got)


@pytest.mark.parametrize("t", GEMM_TYPES)
def test_gemm_ldy_and_split_invariance(Q, oracle, t):
    """prefill mode: every batch size takes the GEMM (one row included) and a token's sums do not depend on
    how the prompt was cut (the reference's qmatvec_set_prefill contract, src/qmatvec.h:43-49)"""
    N, K = 320, 1024
    W = oracle.quantize(t, synth.gaussian(5, N * K, 0, 0.02).reshape(N, K))
    Wd = dev(W)
    x = acts(6, 150, K)
    Q.lib().qmatvec_set_prefill(1)
    try:
        full = run_batch(Q, t, Wd, x, N, K, ldy=N + 13)
        cuts = ((0, 1), (1, 65), (65, 70), (70, 150))  # 64-token workgroups up to 64 tokens, 128 above
        parts = np.concatenate([run_batch(Q, t, Wd, x[s:e], N, K) for s, e in cuts])
    finally:
        Q.lib().qmatvec_set_prefill(0)
    assert np.array_equal(full.view(np.uint32), parts.view(np.uint32))
    check_tokens(oracle, t, W, N, K, x[:3], full[:3])


@pytest.mark.parametrize("t,N,K", [(100, 768, 2048), (100, 2048, 768), (8, 512, 1024), (101, 256, 1024),
                                   (12, 768, 2048), (13, 512, 1024), (14, 2048, 768), (23, 512, 1024),
                                   (39, 256, 1024), (40, 768, 2048), (12, 200, 512)])
def test_moe_tiled_gemm(Q, oracle, t, N, K):
    """expert tiles from the grouping (config 4 shapes, and K-quant experts): entry i of tile k multiplies input
    row in_rows[i] by expert tile_e[k] into output row out_rows[i]"""
    import torch
    E, n_used, T = 16, 4, 48
    W = oracle.quantize(t, synth.gaussian(9, E * N * K, 0, 0.02).reshape(E * N, K))
    ids = (synth.splitmix64(10, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    tile = Q.lib().qmatvec_id_batch_tile(t, N, K)
    assert tile >= 64
    g = oracle.moe_group(ids, E, min(tile, 16))  # small tiles: several tiles per expert
    x = acts(11, T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    y = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
    nt = np.array([g["n_tiles"]], np.int32)
    L = Q.lib()
    import ctypes as C
    p = lambda a: C.c_void_p(a.data_ptr())
    bufs = [dev(nt), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]), dev(g["tok_rows"]),
            dev(g["pair_rows"])]
    rc = L.qmatvec_launch_q8_id_batch(t, p(dev(W)), Q.row_size(t, K), q.ref, p(y), N, K, g["n_tiles"] + 3,
                                      min(tile, 16), *[p(b) for b in bufs], None)
    assert rc == 0
    got = host(y)
    rb = W.shape[1]
    for tt in range(T):
        a = oracle.quantize_act(x[tt], t in (12, 13, 14, 23))
        for j in range(n_used):
            want, ref, mag = oracle.matvec(t, W.reshape(E, N, rb)[ids[tt, j]], N, K, a)
            parity.check(f"expert-tiled GEMM {Q.NAMES[t]}", got[tt * n_used + j], want, mag, ref, TOL)


@pytest.mark.parametrize("t,N,K", [(12, 768, 2048), (14, 2048, 768), (13, 256, 1024), (23, 512, 1024)])
def test_moe_tiled_gemm_kquant_tiles(Q, oracle, t, N, K):
    """the K-quant expert GEMM's 128-entry tiles (the launch's 128-token form, experts of ~150 entries: a full tile
    and a partial one each) against 64-entry tiles (the 64-token form) and 16-entry ones: every entry's output bit for
    bit the same (the same per-super-block integers and epilogue order), and within 1e-5 sum |w x| of the oracle"""
    import ctypes as C
    import torch
    L = Q.lib()
    assert L.qmatvec_id_batch_tile(t, N, K) == 128
    E, n_used, T = 4, 4, 150
    W = oracle.quantize(t, synth.gaussian(90 + t, E * N * K, 0, 0.02).reshape(E * N, K))
    Wd = dev(W)
    ids = (synth.splitmix64(91, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    x = acts(92, T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    p = lambda a: C.c_void_p(a.data_ptr())
    outs = {}
    for tile in (128, 64, 16):
        g = oracle.moe_group(ids, E, tile)
        bufs = [dev(np.array([g["n_tiles"]], np.int32)), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]),
                dev(g["tok_rows"]), dev(g["pair_rows"])]
        y = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
        assert L.qmatvec_launch_q8_id_batch(t, p(Wd), Q.row_size(t, K), q.ref, p(y), N, K, g["n_tiles"] + 1, tile,
                                            *[p(b) for b in bufs], None) == 0
        outs[tile] = host(y)
    assert np.isfinite(outs[128]).all()
    for tile in (64, 16):
        assert np.array_equal(outs[128].view(np.uint32), outs[tile].view(np.uint32)), tile
    rb = W.shape[1]
    for tt in range(0, T, 7):
        a = oracle.quantize_act(x[tt], True)
        for j in range(n_used):
            want, ref, mag = oracle.matvec(t, W.reshape(E, N, rb)[ids[tt, j]], N, K, a)
            parity.check(f"expert-tiled GEMM (128-entry tiles) {Q.NAMES[t]}", outs[128][tt * n_used + j], want, mag,
                         ref, TOL)


@pytest.mark.parametrize("t,N,K", [(100, 768, 2048), (101, 256, 1024), (40, 768, 2048), (8, 512, 1024),
                                   (39, 256, 1024), (12, 768, 2048), (13, 512, 1024), (14, 256, 768),
                                   (23, 512, 1024), (100, 200, 512)])
def test_moe_tiled_gemm_pair(Q, oracle, t, N, K):
    """qmatvec_launch_q8_id_batch_pair (gate and up over the same expert tiles in one launch): each output bit for
    bit the single launch's, with per-expert output scales registered on the second matrix only"""
    import ctypes as C
    import torch
    E, n_used, T = 12, 4, 56
    L = Q.lib()
    Wg = dev(oracle.quantize(t, synth.gaussian(80 + t, E * N * K, 0, 0.02).reshape(E * N, K)))
    Wu = dev(oracle.quantize(t, synth.gaussian(81 + t, E * N * K, 0, 0.02).reshape(E * N, K)))
    ids = (synth.splitmix64(82, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    tile = L.qmatvec_id_batch_tile(t, N, K)
    g = oracle.moe_group(ids, E, tile)
    x = acts(83, T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    p = lambda a: C.c_void_p(a.data_ptr())
    bufs = [dev(np.array([g["n_tiles"]], np.int32)), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]),
            dev(g["tok_rows"]), dev(g["pair_rows"])]
    rb, mt = Q.row_size(t, K), g["n_tiles"] + 2
    nan = lambda: torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
    es = torch.tensor([0.5 + 0.125 * e for e in range(E)], dtype=torch.float32).pin_memory()
    owner = C.c_void_p(0x7F)
    assert L.qmatvec_set_out_scale(owner, p(Wu), Wu.numel(), p(es), E) == 0
    try:
        yg, yu = nan(), nan()
        assert L.qmatvec_launch_q8_id_batch(t, p(Wg), rb, q.ref, p(yg), N, K, mt, tile, *[p(b) for b in bufs],
                                            None) == 0
        assert L.qmatvec_launch_q8_id_batch(t, p(Wu), rb, q.ref, p(yu), N, K, mt, tile, *[p(b) for b in bufs],
                                            None) == 0
        pg, pu = nan(), nan()
        assert L.qmatvec_launch_q8_id_batch_pair(t, p(Wg), p(Wu), rb, q.ref, p(pg), p(pu), N, K, mt, tile,
                                                 *[p(b) for b in bufs], None) == 0
        a, b, c, d = host(yg), host(yu), host(pg), host(pu)
    finally:
        L.qmatvec_drop_out_scales(owner)
    assert np.isfinite(a).all() and np.isfinite(b).all()
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
    assert np.array_equal(b.view(np.uint32), d.view(np.uint32))


@pytest.mark.parametrize("t,N,K", [(100, 768, 2048), (101, 256, 1024), (40, 768, 2048), (100, 384, 512)])
def test_moe_tiled_gemm_swiglu(Q, oracle, t, N, K):
    """qmatvec_launch_q8_id_batch_swiglu (the gate / up pair with SwiGLU and its Q8_0 quantization in the epilogue):
    q0, d0 and s0 of every entry's row bit for bit those of the pair launch followed by gpu_swiglu, with per-expert
    output scales on both matrices and tiles with padding entries"""
    import ctypes as C
    import torch
    from purhie_amd import moe as M
    E, n_used, T = 12, 4, 56
    L = Q.lib()
    assert L.qmatvec_q8_id_batch_swiglu_supported(t, N, K) == 1
    Wg = dev(oracle.quantize(t, synth.gaussian(90 + t, E * N * K, 0, 0.02).reshape(E * N, K)))
    Wu = dev(oracle.quantize(t, synth.gaussian(91 + t, E * N * K, 0, 0.02).reshape(E * N, K)))
    ids = (synth.splitmix64(92, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    tile = L.qmatvec_id_batch_tile(t, N, K)
    g = oracle.moe_group(ids, E, tile)
    x = acts(93, T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    p = lambda a: C.c_void_p(a.data_ptr())
    bufs = [dev(np.array([g["n_tiles"]], np.int32)), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]),
            dev(g["tok_rows"]), dev(g["pair_rows"])]
    rb, mt, R = Q.row_size(t, K), g["n_tiles"] + 2, T * n_used
    owners = (C.c_void_p(0x81), C.c_void_p(0x82))
    es = [torch.tensor([0.5 + 0.125 * ((e * (m + 3)) % E) for e in range(E)], dtype=torch.float32).pin_memory()
          for m in range(2)]
    for o, W, s in zip(owners, (Wg, Wu), es):
        assert L.qmatvec_set_out_scale(o, p(W), W.numel(), p(s), E) == 0
    try:
        yg = torch.full((R, N), float("nan"), device="cuda")
        yu = torch.full((R, N), float("nan"), device="cuda")
        assert L.qmatvec_launch_q8_id_batch_pair(t, p(Wg), p(Wu), rb, q.ref, p(yg), p(yu), N, K, mt, tile,
                                                 *[p(b) for b in bufs], None) == 0
        want = Q.Q8(R * N)
        h = torch.zeros(R * N, device="cuda")
        assert M.lib().gpu_swiglu(p(yg), p(yu), p(h), R * N, want.ref, None) == 0
        got = Q.Q8(R * N)
        got.mem.fill_(0x5A)  # every byte the launch owns must be written
        assert L.qmatvec_launch_q8_id_batch_swiglu(t, p(Wg), p(Wu), rb, q.ref, got.ref, N, K, mt, tile,
                                                   *[p(b) for b in bufs], None) == 0
        torch.cuda.synchronize()
    finally:
        for o in owners:
            L.qmatvec_drop_out_scales(o)
    a, b = want.views(R * N), got.views(R * N)
    assert torch.isfinite(a["d0"]).all() and (a["d0"] != 0).any()
    for f in ("q0", "d0", "s0"):
        assert torch.equal(a[f].view(torch.uint8), b[f].view(torch.uint8)), f


def test_moe_tiled_gemm_swiglu_refused(Q):
    L = Q.lib()
    assert L.qmatvec_q8_id_batch_swiglu_supported(12, 768, 2048) == 0  # a K-quant: no split GEMM
    assert L.qmatvec_q8_id_batch_swiglu_supported(100, 200, 2048) == 0  # N % 128
    assert L.qmatvec_q8_id_batch_swiglu_supported(100, 768, 2048) == 1


@pytest.fixture(params=["tile", "wave"])
def kpath(request, monkeypatch):
    """the decode kernels under test: the one-unit-per-lane tile kernels or the per-wave kernels"""
    from purhie_amd import qmatvec
    prev = qmatvec.decode_path(1 if request.param == "tile" else 0)
    yield request.param
    qmatvec.decode_path(prev)


@pytest.fixture
def fp32_mode(Q):
    """prefill-fp32 mode (qmatvec_set_prefill_fp32, src/qmatvec.cpp:49-52): the MFMA GEMMs off"""
    Q.lib().qmatvec_set_prefill_fp32(1)
    yield
    Q.lib().qmatvec_set_prefill_fp32(0)


def single_token(Q, t, Wd, x, N, K):
    """each token alone through the decode matvec"""
    import torch
    out = np.empty((x.shape[0], N), np.float32)
    q = Q.Q8(((K + 255) // 256) * 256)
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    for i in range(x.shape[0]):
        Q.quantize(dev(x[i]), K, q)
        Q.launch_q8(t, Wd, q, y, N, K)
        out[i] = host(y)
    return out


@pytest.mark.parametrize("t", GEMM_TYPES)
def test_prefill_fp32_mode_decode_order(Q, oracle, kpath, fp32_mode, t):
    """with the MFMA GEMMs off, a 40-token batch (the GEMM's size otherwise) equals its tokens' single-token
    decode bit for bit"""
    N, K, T = 320, 1024, 40
    W = oracle.quantize(t, synth.gaussian(21, N * K, 0, 0.02).reshape(N, K))
    Wd = dev(W)
    x = acts(22, T, K)
    got = run_batch(Q, t, Wd, x, N, K)
    want = single_token(Q, t, Wd, x, N, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,N,K", [(100, 768, 2048), (12, 256, 768), (14, 256, 768), (8, 96, 1024)])
def test_moe_tiles_decode_order(Q, oracle, kpath, fp32_mode, t, N, K):
    """with the MFMA GEMMs off, the expert tiles (the reference's tile of 16) run through the decode kernels: every
    entry equals the single-token decode of its expert bit for bit"""
    import ctypes as C
    import torch
    E, n_used, T = 8, 4, 20
    rb = Q.row_size(t, K)
    W = oracle.quantize(t, synth.gaussian(23, E * N * K, 0, 0.02).reshape(E * N, K))
    Wd = dev(W)
    ids = (synth.splitmix64(24, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    L = Q.lib()
    tile = L.qmatvec_id_batch_tile(t, N, K)
    assert tile == 16
    g = oracle.moe_group(ids, E, tile)
    x = acts(25, T, K)
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    y = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
    p = lambda a: C.c_void_p(a.data_ptr())
    bufs = [dev(np.array([g["n_tiles"]], np.int32)), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]),
            dev(g["tok_rows"]), dev(g["pair_rows"])]
    rc = L.qmatvec_launch_q8_id_batch(t, p(Wd), rb, q.ref, p(y), N, K, g["n_tiles"] + 2, tile,
                                      *[p(b) for b in bufs], None)
    assert rc == 0
    got = host(y)
    for e in range(E):
        sel = [(tt, j) for tt in range(T) for j in range(n_used) if ids[tt, j] == e]
        if not sel:
            continue
        We = Wd[e * N:(e + 1) * N]  # expert e's N rows of rb bytes
        assert We.numel() == N * rb and We.is_contiguous()
        want = single_token(Q, t, We, x[[tt for tt, _ in sel]], N, K)
        for r, (tt, j) in enumerate(sel):
            assert np.array_equal(got[tt * n_used + j].view(np.uint32), want[r].view(np.uint32)), (e, tt, j)
