"""The hot kernels' own integer sums, bit for bit against the oracle (capture mode, qmatvec_debug_capture).

In capture mode a launch runs its kernel's capture instantiation: the same decode and v_dot4 / MFMA code as the
production kernel, which also adds every integer sum it forms into a buffer. The decode kernels (tile and per-wave,
dense, few-token, expert-indexed and SwiGLU-fused) expose each weight scale group's dot (north_star: "bit-exact
per-block int32 dot sums"); the K-quant GEMM exposes each super-block's isum = sum_j sc_j dot_j. The oracle's
block dots are pinned by brute force on decoded values, its super-block isum by decoded weights
(tests/test_oracle.py). Weights are random block bytes: the integer sums depend only on the levels and scales,
and random bytes reach every level and scale byte.
"""
import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu
KQ = (12, 13, 14, 23)


@pytest.fixture(scope="module")
def Q():
    from purhie_amd import qmatvec
    qmatvec.lib()
    yield qmatvec
    qmatvec.lib().qmatvec_set_prefill(0)


@pytest.fixture(params=["tile", "wave"])
def kpath(request, Q):
    prev = Q.decode_path(1 if request.param == "tile" else 0)
    yield request.param
    Q.decode_path(prev)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rand_rows(Q, t, N, K, seed):
    """N rows of random block bytes (Q6_K's fp16 d included: the integer sums never read it)"""
    rb = Q.row_size(t, K)
    return (synth.splitmix64(seed, N * rb) & np.uint64(0xFF)).astype(np.uint8).reshape(N, rb)


def acts(seed, T, K):
    x = synth.gaussian(seed, T * K)
    x = synth.with_outliers(x, seed + 1, 0.001, 20.0)
    return x.reshape(T, K)


def quantized(Q, x):
    T, K = x.shape
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    return q


def cap_buf(n):
    import torch
    return torch.zeros(n, dtype=torch.int32, device="cuda")


# the configs' shapes (1: Q8_0 3072x1024; 2: Q4_K 9728x2560 and 2560x9728 at T = 1 and 4; 4: ROCmFP4 expert
# gate / down), the mixed-quant expert shapes, and the other formats
DECODE = [(8, 3072, 1024, 1), (12, 9728, 2560, 1), (12, 2560, 9728, 1), (12, 9728, 2560, 4), (12, 2560, 9728, 4),
          (100, 768, 2048, 1), (100, 2048, 768, 1), (100, 17408 // 8, 5120, 2), (101, 768, 2048, 3),
          (14, 2048, 1024, 1), (14, 3072, 1024, 4), (13, 1024, 2560, 2), (23, 1024, 2560, 1), (39, 768, 2048, 2),
          (40, 768, 2048, 1), (8, 2048, 3072, 4),
          # tokens whose activation passes the tile's LDS: staged a few at a time (Q8_0 two passes of 2, Q6_K three
          # of 1, ROCmFP4 two of 1)
          (8, 512, 8192, 4), (14, 300, 5120, 3), (100, 256, 12288, 2)]


@pytest.mark.parametrize("t,N,K,T", DECODE)
def test_decode_block_dots(Q, oracle, kpath, t, N, K, T):
    W = rand_rows(Q, t, N, K, 100 + t + N + K)
    x = acts(200 + T + K, T, K)
    q = quantized(Q, x)
    G = Q.capture_unit(t)
    cap = cap_buf(T * N * (K // G))
    import torch
    y = torch.zeros((T, N), dtype=torch.float32, device="cuda")
    with Q.capture(cap):
        if T == 1:
            Q.launch_q8(t, dev(W), q, y, N, K)
        else:
            Q.launch_q8_multi_t(t, [dev(W)], [N], [y], q, K, T)
    got = host(cap).reshape(T, N, K // G)
    for i in range(T):
        a = oracle.quantize_act(x[i], t in KQ)
        assert np.array_equal(got[i], oracle.block_dots(t, W, N, K, a["q"])), f"token {i}"


@pytest.mark.parametrize("t", (12, 100))
def test_decode_block_dots_pair_and_batch(Q, oracle, kpath, t):
    """the pair launch (rows of W, then W2) and a 6-token batch below the GEMM threshold (groups of 4 + 2)"""
    import torch
    K = 2560 if t == 12 else 2048
    N1, N2, T = 700, 300, 6
    W1, W2 = rand_rows(Q, t, N1, K, 31), rand_rows(Q, t, N2, K, 32)
    x = acts(33, T, K)
    G = Q.capture_unit(t)
    L = Q.lib()
    import ctypes as C
    p = lambda a: C.c_void_p(a.data_ptr())
    q1 = quantized(Q, x[:1])
    cap = cap_buf((N1 + N2) * (K // G))
    y1, y2 = torch.zeros(N1, device="cuda"), torch.zeros(N2, device="cuda")
    with Q.capture(cap):
        assert L.qmatvec_launch_q8_pair(t, p(dev(W1)), N1, p(y1), p(dev(W2)), N2, p(y2), Q.row_size(t, K), q1.ref, K,
                                        None) == 0
    a = oracle.quantize_act(x[0], t in KQ)
    got = host(cap).reshape(N1 + N2, K // G)
    assert np.array_equal(got[:N1], oracle.block_dots(t, W1, N1, K, a["q"]))
    assert np.array_equal(got[N1:], oracle.block_dots(t, W2, N2, K, a["q"]))
    qT = quantized(Q, x)
    cap = cap_buf(T * N1 * (K // G))
    y = torch.zeros((T, N1), device="cuda")
    with Q.capture(cap):
        Q.launch_q8_batch(t, dev(W1), qT, y, N1, N1, K, T)
    got = host(cap).reshape(T, N1, K // G)
    for i in range(T):
        a = oracle.quantize_act(x[i], t in KQ)
        assert np.array_equal(got[i], oracle.block_dots(t, W1, N1, K, a["q"])), f"token {i}"


@pytest.mark.parametrize("t,N,K", [(100, 768, 2048), (12, 1024, 3072), (14, 3072, 1024), (8, 512, 2048),
                                   (101, 768, 2048)])
def test_expert_block_dots(Q, oracle, kpath, t, N, K):
    """expert-indexed pair launch (config 4 / 5 decode: gate + up, id -1 = the extra matrices): layout
    [matrix][output row][row][group]"""
    import torch
    E, n_used, T = 12, 4, 2
    W, W2 = rand_rows(Q, t, E * N, K, 41), rand_rows(Q, t, E * N, K, 42)
    Wx, W2x = rand_rows(Q, t, N, K, 43), rand_rows(Q, t, N, K, 44)
    ids = np.array([[3, 0, -1, 11], [7, 3, 5, 1]], dtype=np.int32)
    x = acts(45, T, K)
    q = quantized(Q, x)
    G = Q.capture_unit(t)
    cap = cap_buf(2 * T * n_used * N * (K // G))
    y = torch.zeros((T * n_used, N), device="cuda")
    y2 = torch.zeros((T * n_used, N), device="cuda")
    with Q.capture(cap):
        Q.launch_q8_id_x(t, dev(W), dev(W2), dev(Wx), dev(W2x), dev(ids), n_used, 0, q, y, y2, N, K, T)
    got = host(cap).reshape(2, T * n_used, N, K // G)
    rb = W.shape[1]
    for tt in range(T):
        a = oracle.quantize_act(x[tt], t in KQ)
        for j in range(n_used):
            e = ids[tt, j]
            for m, (M, Mx) in enumerate(((W, Wx), (W2, W2x))):
                rows = Mx if e < 0 else M.reshape(E, N, rb)[e]
                assert np.array_equal(got[m, tt * n_used + j], oracle.block_dots(t, rows, N, K, a["q"]))


@pytest.mark.parametrize("t", (100, 101, 8))
def test_swiglu_fused_block_dots(Q, oracle, t):
    """the expert down matvec with SwiGLU and its Q8_0 quantization folded in (config 4 decode): its dots equal the
    oracle's on the activation gpu_swiglu quantizes (read back), for every slot"""
    import ctypes as C
    import torch
    from purhie_amd import moe as M
    E, n_used, N, K = 16, 8, 2048, 768
    W = rand_rows(Q, t, E * N, K, 51)
    Wx = rand_rows(Q, t, N, K, 52)
    ids = np.array([[5, 0, 9, -1, 15, 2, 7, 3]], dtype=np.int32)
    g = dev(synth.gaussian(53, n_used * K).reshape(n_used, K))
    u = dev(synth.gaussian(54, n_used * K).reshape(n_used, K))
    p = lambda a: None if a is None else C.c_void_p(a.data_ptr())
    G = Q.capture_unit(t)
    cap = cap_buf(n_used * N * (K // G))
    y = torch.zeros((n_used, N), device="cuda")
    L = Q.lib()
    with Q.capture(cap):
        assert L.qmatvec_launch_q8_id_swiglu(t, p(dev(W)), p(dev(Wx)), Q.row_size(t, K), p(dev(ids)), n_used, p(g),
                                             p(u), p(y), N, K, 1, None) == 0
    got = host(cap).reshape(n_used, N, K // G)
    qa = Q.Q8(n_used * K)
    h = torch.zeros(n_used * K, device="cuda")
    assert M.lib().gpu_swiglu(p(g), p(u), p(h), n_used * K, qa.ref, None) == 0
    q0 = host(qa.views(n_used * K)["q0"]).reshape(n_used, K)
    rb = W.shape[1]
    for j in range(n_used):
        e = ids[0, j]
        rows = Wx if e < 0 else W.reshape(E, N, rb)[e]
        assert np.array_equal(got[j], oracle.block_dots(t, rows, N, K, q0[j])), f"slot {j}"


@pytest.mark.parametrize("t,N,K,T", [(12, 9728 // 8, 2560, 200), (12, 300, 9728, 70), (13, 256, 1024, 130),
                                     (14, 3072 // 4, 1024, 129), (23, 256, 2048, 64)])
def test_kquant_gemm_isum(Q, oracle, t, N, K, T):
    """the K-quant prefill GEMM's exact per-super-block integer isum (prefill mode: every T takes the GEMM), for
    the tokens of a partial last tile too"""
    import torch
    assert Q.capture_unit(t, gemm=True) == 256
    W = rand_rows(Q, t, N, K, 61 + t)
    x = acts(62 + T, T, K)
    q = quantized(Q, x)
    cap = cap_buf(T * N * (K // 256))
    y = torch.zeros((T, N), device="cuda")
    Q.lib().qmatvec_set_prefill(1)
    try:
        with Q.capture(cap):
            Q.launch_q8_batch(t, dev(W), q, y, N, N, K, T)
    finally:
        Q.lib().qmatvec_set_prefill(0)
    got = host(cap).reshape(T, N, K // 256)
    for i in range(T):
        a = oracle.quantize_act(x[i], True)
        assert np.array_equal(got[i], oracle.unit_isum(t, W, N, K, a["q"], a["bs"])), f"token {i}"


@pytest.mark.parametrize("t,N,K", [(12, 768, 2048), (14, 2048, 768)])
@pytest.mark.parametrize("tile", [128, 64])
def test_kquant_expert_gemm_isum(Q, oracle, t, N, K, tile):
    """the K-quant expert-tiled GEMM's per-super-block integers at both launch forms (128- and 64-entry tiles; the
    mixed-quant MoE's gate and down shapes), per entry's output row"""
    import ctypes as C
    import torch
    E, n_used, T = 4, 4, 100
    W = rand_rows(Q, t, E * N, K, 71 + t)
    ids = (synth.splitmix64(72, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    x = acts(73, T, K)
    q = quantized(Q, x)
    g = oracle.moe_group(ids, E, tile)
    p = lambda a: C.c_void_p(a.data_ptr())
    bufs = [dev(np.array([g["n_tiles"]], np.int32)), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]),
            dev(g["tok_rows"]), dev(g["pair_rows"])]
    cap = cap_buf(T * n_used * N * (K // 256))
    y = torch.zeros((T * n_used, N), device="cuda")
    with Q.capture(cap):
        assert Q.lib().qmatvec_launch_q8_id_batch(t, p(dev(W)), Q.row_size(t, K), q.ref, p(y), N, K,
                                                  g["n_tiles"] + 1, tile, *[p(b) for b in bufs], None) == 0
    got = host(cap).reshape(T * n_used, N, K // 256)
    rb = W.shape[1]
    for tt in range(0, T, 9):
        a = oracle.quantize_act(x[tt], True)
        for j in range(n_used):
            rows = W.reshape(E, N, rb)[ids[tt, j]]
            assert np.array_equal(got[tt * n_used + j], oracle.unit_isum(t, rows, N, K, a["q"], a["bs"])), (tt, j)


def test_capture_units(Q):
    """the group each decode capture holds is the weight scale's; the GEMMs' units: a K-quant super-block, a Q8_0 /
    MXFP4 block, and none for the split GEMM of ROCmFP4 / FAST / NVFP4 (exact fp16 operands chained through K)"""
    for t, g in {8: 32, 100: 16, 101: 32, 12: 32, 13: 32, 14: 16, 23: 32, 39: 32, 40: 16}.items():
        assert Q.capture_unit(t) == g
    for t in KQ:
        assert Q.capture_unit(t, gemm=True) == 256
    for t in (8, 39):
        assert Q.capture_unit(t, gemm=True) == 32
    for t in (100, 101, 40):
        assert Q.capture_unit(t, gemm=True) == 0
    assert Q.capture_unit(1) == 0


def test_capture_capacity_error(Q):
    """a launch whose capture would not fit the buffer is refused (hipErrorInvalidValue) before it runs"""
    import torch
    t, N, K = 12, 64, 512
    W = rand_rows(Q, t, N, K, 71)
    q = quantized(Q, acts(72, 1, K))
    y = torch.zeros(N, device="cuda")
    cap = cap_buf(N * (K // 32) - 1)
    L = Q.lib()
    import ctypes as C
    with Q.capture(cap):
        rc = L.qmatvec_launch_q8(t, C.c_void_p(dev(W).data_ptr()), Q.row_size(t, K), q.ref, C.c_void_p(y.data_ptr()),
                                 N, K, None)
    assert rc == 1


@pytest.mark.parametrize("t,N,K,T", [(8, 300, 1024, 150), (8, 2048, 2048, 40), (39, 256, 2048, 70)])
def test_block_gemm_dots(Q, oracle, t, N, K, T):
    """the per-block int8 GEMM (Q8_0, MXFP4; prefill mode): each 32-value block's exact int32 dot, the integer its
    epilogue scales by e_w d_x"""
    import torch
    assert Q.capture_unit(t, gemm=True) == 32
    W = rand_rows(Q, t, N, K, 81 + t)
    x = acts(82 + T, T, K)
    q = quantized(Q, x)
    cap = cap_buf(T * N * (K // 32))
    y = torch.zeros((T, N), device="cuda")
    Q.lib().qmatvec_set_prefill(1)
    try:
        with Q.capture(cap):
            Q.launch_q8_batch(t, dev(W), q, y, N, N, K, T)
    finally:
        Q.lib().qmatvec_set_prefill(0)
    got = host(cap).reshape(T, N, K // 32)
    for i in range(T):
        a = oracle.quantize_act(x[i], False)
        assert np.array_equal(got[i], oracle.block_dots(t, W, N, K, a["q"])), f"token {i}"
