"""fp32 activations over quantized weights (qmatvec_launch, qmatvec_launch_batch for Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS,
MXFP4, NVFP4, ROCmFP4 and ROCmFP4_FAST; qmatvec_launch_id and qmatvec_launch_id_batch_f for those and F32 / F16 /
BF16; reference src/qmatvec.cpp:255-367,601-671, src/matvec_q.hip:640-717,1076-1237):
- every output within 1e-5 * sum |w x| of the double sum over the oracle's decoded weights (the oracle's decoder is
  pinned to the compiled reference's qt_to_float) and the fp32 activations: the reference's criterion
  (tests/matvec_verify.cpp:117-145);
- a batch the same bits as its tokens one by one;
- each expert-indexed output the same bits as the dense launch on that expert's rows and input row (both slot
  conventions), an id of -1 writing nothing;
- each expert-tile entry the same bits as the expert-indexed launch;
- a registered output scale (one per matrix, or one per stacked expert) multiplies the sums, rounded once;
- the reference's error codes."""
import ctypes as C

import numpy as np
import pytest

from purhie_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
QUANT = {8: "q8_0", 12: "q4_K", 13: "q5_K", 14: "q6_K", 23: "iq4_xs", 39: "mxfp4", 40: "nvfp4", 100: "rocmfp4",
         101: "rocmfp4_fast"}
F32, F16, BF16 = 0, 1, 30


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


def weights(oracle, t, seed, N, K):
    """N x K ~N(0, 0.05) as type t's bytes (the oracle's encoder for the quantized types)"""
    w = synth.gaussian(seed, N * K, 0, 0.05).reshape(N, K)
    if t in QUANT:
        return oracle.quantize(t, w)
    if t == F32:
        return w.view(np.uint8).reshape(N, -1)
    if t == F16:
        return w.astype(np.float16).view(np.uint8).reshape(N, -1)
    u = w.view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8).reshape(N, -1)


def decoded(oracle, t, W, K):
    if t in QUANT:
        return oracle.to_float(t, W, K).astype(np.float64)
    if t == F32:
        return W.view(np.float32).reshape(-1, K).astype(np.float64)
    if t == F16:
        return W.view(np.float16).reshape(-1, K).astype(np.float64)
    return (W.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(-1, K).astype(np.float64)


def acts(seed, T, K):
    x = synth.gaussian(seed, T * K).reshape(T, K)
    x[:, ::97] *= 30.0  # a few large values
    return x


def check(Wd64, x, got):
    ref = x.astype(np.float64) @ Wd64.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(Wd64).T
    err = np.abs(got.astype(np.float64) - ref) / (mag + 1e-30)
    assert err.max() <= TOL, f"max rel err {err.max():.3g}"


def ks(t):
    return (768, 2048) if t in (12, 13, 14, 23) else (512, 2048)


@pytest.mark.parametrize("t", sorted(QUANT))
def test_supported(Q, t):
    L = Q.lib()
    assert L.qmatvec_supported(t) == 1 and L.qmatvec_id_batch_f_supported(t) == 1


@pytest.mark.parametrize("t", sorted(QUANT))
def test_decode_and_batch(Q, oracle, t):
    """one token against the oracle; a 9-token batch the same bits as its tokens alone"""
    import torch
    L = Q.lib()
    for K in ks(t):
        N, T = 301, 9
        W = weights(oracle, t, 10 + K + t, N, K)
        Wd, rb = dev(W), W.shape[1]
        x = acts(20 + K, T, K)
        xd = dev(x)
        y1 = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
        for i in range(T):
            assert L.qmatvec_launch(t, p(Wd), rb, C.c_void_p(xd.data_ptr() + 4 * i * K),
                                    C.c_void_p(y1.data_ptr() + 4 * i * N), N, K, None) == 0
        yb = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
        assert L.qmatvec_launch_batch(t, p(Wd), rb, p(xd), p(yb), N, K, T, None) == 0
        got1, gotb = host(y1), host(yb)
        check(decoded(oracle, t, W, K), x, got1)
        assert np.array_equal(got1.view(np.uint32), gotb.view(np.uint32)), (t, K)


def expert_case(oracle, t, E, N, K, seed):
    W = np.concatenate([weights(oracle, t, seed + e, N, K) for e in range(E)])
    return W, W.shape[1]


@pytest.mark.parametrize("t", sorted(QUANT) + [F32, F16, BF16])
@pytest.mark.parametrize("x_per_slot", (0, 1))
def test_expert_indexed(Q, oracle, t, x_per_slot):
    """each (token, slot) output equals the dense launch on its expert's rows and input row, bit for bit; an id of
    -1 leaves its output row as it was"""
    import torch
    L = Q.lib()
    E, N, n_used, T = 5, 67, 3, 4
    K = ks(t)[0] if t in QUANT else 200
    W, rb = expert_case(oracle, t, E, N, K, 50 + t)
    Wd = dev(W)
    ids = np.array([[4, 0, 2], [1, -1, 4], [3, 3, 0], [2, 1, -1]], np.int32)
    nx = T * n_used if x_per_slot else T
    x = acts(60 + t, nx, K)
    xd = dev(x)
    y = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_id(t, p(Wd), rb, p(dev(ids)), n_used, x_per_slot, p(xd), p(y), N, K, T, None) == 0
    got = host(y)
    Wdec = decoded(oracle, t, W, K)
    for tt in range(T):
        for j in range(n_used):
            e, r = int(ids[tt, j]), tt * n_used + j
            if e < 0:
                assert np.isnan(got[r]).all()
                continue
            xi = r if x_per_slot else tt
            if t in QUANT:
                one = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
                assert L.qmatvec_launch(t, C.c_void_p(Wd.data_ptr() + e * N * rb), rb,
                                        C.c_void_p(xd.data_ptr() + 4 * xi * K), p(one), N, K, None) == 0
                assert np.array_equal(host(one).view(np.uint32), got[r].view(np.uint32)), (tt, j)
            check(Wdec[e * N:(e + 1) * N], x[xi:xi + 1], got[r][None])


def tiles_of(ids, n_used, x_per_slot, tile):
    """the (token, slot) entries grouped by expert into tiles of up to `tile` (a host grouping in the reference's
    tile convention: in_rows index the input, out_rows the output)"""
    T = ids.shape[0]
    te, ts, tn, inr, outr = [], [], [], [], []
    for e in sorted(set(ids.reshape(-1).tolist()) - {-1}):
        ent = [(tt, j) for tt in range(T) for j in range(n_used) if ids[tt, j] == e]
        for i in range(0, len(ent), tile):
            part = ent[i:i + tile]
            te.append(e)
            ts.append(len(inr))
            tn.append(len(part))
            for tt, j in part:
                inr.append(tt * n_used + j if x_per_slot else tt)
                outr.append(tt * n_used + j)
    return [np.array(v, np.int32) for v in (te, ts, tn, inr, outr)]


@pytest.mark.parametrize("t", sorted(QUANT) + [F32, BF16])
def test_expert_tiles_same_bits_as_indexed(Q, oracle, t):
    """expert tiles (up to 16 entries, and a short tile limit) give each entry the expert-indexed launch's bits"""
    import torch
    L = Q.lib()
    E, N, n_used, T = 6, 70, 4, 24
    K = ks(t)[0] if t in QUANT else 256
    W, rb = expert_case(oracle, t, E, N, K, 80 + t)
    Wd = dev(W)
    rng = np.random.default_rng(t)
    ids = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
    ids[rng.integers(0, T, 3), 0] = 2  # one popular expert (more than one tile of it)
    x = acts(90 + t, T, K)
    xd = dev(x)
    ref = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.qmatvec_launch_id(t, p(Wd), rb, p(dev(ids)), n_used, 0, p(xd), p(ref), N, K, T, None) == 0
    want = host(ref)
    for tile in (16, 5):
        te, ts, tn, inr, outr = tiles_of(ids, n_used, 0, tile)
        nt = dev(np.array([len(te)], np.int32))
        y = torch.full((T * n_used, N), float("nan"), dtype=torch.float32, device="cuda")
        assert L.qmatvec_launch_id_batch_f(t, p(Wd), rb, p(xd), p(y), N, K, len(te) + 3, tile, p(nt), p(dev(te)),
                                           p(dev(ts)), p(dev(tn)), p(dev(inr)), p(dev(outr)), None) == 0
        assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32)), tile


@pytest.mark.parametrize("t", (40, 100, 12))
def test_output_scales(Q, oracle, t):
    """a matrix's registered scale, and per-expert scales of stacked experts, multiply the sums (rounded once)"""
    import torch
    L = Q.lib()
    N, K, E = 64, ks(t)[0], 3
    W, rb = expert_case(oracle, t, E, N, K, 110 + t)
    Wd = dev(W)
    x = acts(120, 1, K)
    xd = dev(x)
    owner = C.c_void_p(0x5CA1E)

    def dense():
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        assert L.qmatvec_launch(t, p(Wd), rb, p(xd), p(y), N, K, None) == 0
        return host(y)

    def indexed():
        y = torch.empty((E, N), dtype=torch.float32, device="cuda")
        ids = dev(np.arange(E, dtype=np.int32)[None])
        assert L.qmatvec_launch_id(t, p(Wd), rb, p(ids), E, 0, p(xd), p(y), N, K, 1, None) == 0
        return host(y)

    base, base_id = dense(), indexed()
    s1 = torch.tensor([0.37], dtype=torch.float32).pin_memory()  # (read by the host and the GPU)
    assert L.qmatvec_set_out_scale(owner, p(Wd), N * rb, p(s1), 1) == 0
    try:
        assert np.array_equal(dense().view(np.uint32), (base * np.float32(0.37)).view(np.uint32))
    finally:
        L.qmatvec_drop_out_scales(owner)
    se = np.array([0.5, 3.0, 0.125], np.float32)
    s3 = torch.from_numpy(se).pin_memory()
    assert L.qmatvec_set_out_scale(owner, p(Wd), Wd.numel(), p(s3), E) == 0
    try:
        got = indexed()
    finally:
        L.qmatvec_drop_out_scales(owner)
    assert np.array_equal(got.view(np.uint32), (base_id * se[:, None]).astype(np.float32).view(np.uint32))
    assert np.array_equal(dense().view(np.uint32), base.view(np.uint32))


def test_error_codes(Q):
    import torch
    L = Q.lib()
    W = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    x = torch.zeros(4096, dtype=torch.float32, device="cuda")
    y = torch.zeros(4096, dtype=torch.float32, device="cuda")
    ids = torch.zeros(8, dtype=torch.int32, device="cuda")
    assert L.qmatvec_launch(12, p(W), 144, p(x), p(y), 4, 255, None) == 1            # K not whole super-blocks
    assert L.qmatvec_launch(100, p(W), 17 * 2, p(x), p(y), 4, 64, None) == 1         # row bytes of FAST, not ROCmFP4
    assert L.qmatvec_launch_batch(8, p(W), 34 * 2, p(x), p(y), 4, 64, 0, None) == 1  # T < 1
    assert L.qmatvec_launch_id(8, p(W), 34 * 2, p(ids), 0, 0, p(x), p(y), 4, 64, 1, None) == 1  # n_used 0
    assert L.qmatvec_launch_id(2, p(W), 18 * 2, p(ids), 1, 0, p(x), p(y), 4, 64, 1, None) == 98  # no Q4_0 kernel
    assert L.qmatvec_launch_id_batch_f(8, p(W), 34 * 2, p(x), p(y), 4, 64, 1, 17, p(ids), p(ids), p(ids), p(ids),
                                       p(ids), p(ids), None) == 1                     # tile > 16
    assert L.qmatvec_launch(8, p(W), 34 * 2, p(x), p(y), 0, 64, None) == 0           # no rows: nothing to do
