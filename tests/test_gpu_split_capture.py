"""The split GEMM's operands bit for bit (capture mode): ROCmFP4, FAST and NVFP4 prefill on fp16 MFMA.

The split GEMM (gemm_split.hip: configs[2]'s prefill and configs[3]'s expert tiles) forms no integer block sums:
it hands the matrix core exact fp16 operands and accumulates their products in fp32 straight through K. Its
exactness therefore rests on the operands, which capture mode exposes from the production kernel's own code (the
same staging, decode and split; the capture instantiation only stores what it formed):
- each staged weight block, which must equal the oracle's decode CB[code] * UE4M3 half-scale (FAST, NVFP4: their
  codebooks and scales) bit for bit: the value is exact in fp16;
- each token's per-row power of two s, which must be 14 minus the exponent of 127 * max_b d0 (clamped to +-100);
- each token's hi and lo planes, whose sum must equal q0 * d0 * 2^s exactly (the lo plane is the exact remainder).
With exact operands, the products are exact in fp32 and only the fp32 accumulation order differs from the
reference's per-block float sums; that part is the tolerance the output tests (test_gpu_fullsize.py,
test_gpu_gemm.py) check. Reference: src/matvec_q.hip:2566-2973 (the WMMA kernels this one replaces),
src/quant_types.cpp:349-382 (the decoders), src/q8_device.h:54-104 (the Q8_0 activation).
"""
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


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def p(t):
    return C.c_void_p(t.data_ptr())


def layout(K, XR):
    """gemm_split_capture_layout (purhie_amd/csrc/kernels.h), in int32 units"""
    plane = XR * (K // 32) * 16
    return dict(lo=plane, s=2 * plane, w=2 * plane + (XR + 3) // 4 * 4)


def cap_ints(K, XR, wrows):
    L = layout(K, XR)
    return L["w"] + wrows * (K // 32) * 16


def check_weights(oracle, t, W, K, cap, L, wrows, rows_seen):
    """staged fp16 weight blocks == the oracle's decode, for the rows the launch staged"""
    nb = K // 32
    got = cap[L["w"]:L["w"] + wrows * nb * 16].view(np.float16).reshape(wrows, K)[rows_seen]
    want = oracle.to_float(t, W[rows_seen], K)
    # equal as numbers: identical bits for every nonzero value; a zero level may carry either sign (the product's
    # sum is the same)
    bad = got.astype(np.float32) != want
    assert not bad.any(), f"{int(bad.sum())} staged weight values differ, first at {np.argwhere(bad)[0]}"


def check_tokens(cap, L, K, q0, d0, rows):
    """the per-row power of two and the exact hi + lo split, for activation rows `rows`"""
    nb = K // 32
    sh = cap[L["s"] + rows].astype(np.int64)
    m = np.max(d0.reshape(-1, nb)[rows], axis=1).astype(np.float32)
    _, ex = np.frexp(np.float32(127.0) * m)
    want_sh = np.clip(np.where(m > 0, 14 - ex, 14), -100, 100)
    assert np.array_equal(sh, want_sh), "per-token power of two"
    plane = lambda off: cap[off:off + len(q0) // K * nb * 16].view(np.float16).reshape(-1, K)[rows]
    hi = plane(0).astype(np.float64)
    lo = plane(L["lo"]).astype(np.float64)
    x = q0.reshape(-1, K)[rows].astype(np.float64) * np.repeat(d0.reshape(-1, nb)[rows].astype(np.float64), 32, axis=1)
    want = x * np.exp2(sh.astype(np.float64))[:, None]
    bad = hi + lo != want
    assert not bad.any(), f"{int(bad.sum())} values with hi + lo != q d0 2^s, first at {np.argwhere(bad)[0]}"
    # hi is the fp16 rounding of the product and lo the remainder's
    assert np.array_equal(hi.astype(np.float16), want.astype(np.float16))


def run_dense(Q, t, Wd, q, N, K, T, XR, cap):
    import torch
    y = torch.zeros((T, N), device="cuda")
    L = Q.lib()
    L.qmatvec_set_prefill(1)
    try:
        with Q.capture(cap):
            assert L.qmatvec_launch_q8_batch(t, p(Wd), Q.row_size(t, K), q.ref, p(y), N, N, K, T, None) == 0
        y0 = torch.zeros((T, N), device="cuda")
        assert L.qmatvec_launch_q8_batch(t, p(Wd), Q.row_size(t, K), q.ref, p(y0), N, N, K, T, None) == 0
    finally:
        L.qmatvec_set_prefill(0)
    return host(y), host(y0)


def quantized(Q, x):
    T, K = x.shape
    q = Q.Q8(((T * K + 255) // 256) * 256)
    Q.quantize(dev(x.reshape(-1)), T * K, q)
    return q


@pytest.mark.parametrize("t,N,K,T", [(100, 1000, 2048, 40), (101, 600, 1024, 200), (40, 520, 2048, 130),
                                     (100, 300, 512, 64)])
def test_split_gemm_operands_dense(Q, oracle, t, N, K, T):
    """dense tiles (64-token tiles of 128 rows up to 64 tokens, 128 x 256 above), partial row and token tiles,
    random block bytes (every code and scale byte)"""
    import torch
    rb = Q.row_size(t, K)
    W = (synth.splitmix64(300 + t, N * rb) & np.uint64(0xFF)).astype(np.uint8).reshape(N, rb)
    x = synth.with_outliers(synth.gaussian(301 + T, T * K), 302, 0.001, 20.0).reshape(T, K)
    q = quantized(Q, x)
    XR = q.max_k // K
    cap = torch.zeros(cap_ints(K, XR, N), dtype=torch.int32, device="cuda")
    y, y0 = run_dense(Q, t, dev(W), q, N, K, T, XR, cap)
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32)), "the capture instantiation's outputs"
    c = host(cap)
    L = layout(K, XR)
    a = oracle.quantize_act(x, False)
    check_weights(oracle, t, W, K, c, L, N, np.arange(N))
    check_tokens(c, L, K, a["q"], a["d"], np.arange(T))


def test_split_gemm_operands_config3(Q, oracle):
    """configs[2] at its own size: ROCmFP4 17408 x 5120 over 2427 tokens with 0.1% outliers x20, weights and
    activations as the benchmark makes them (synth seeds 0x5EED0002, 0x5EED1002, 0x5EED3002)"""
    import torch
    t, N, K, T = 100, 17408, 5120, 2427
    Wd = torch.empty((N, Q.row_size(t, K)), dtype=torch.uint8, device="cuda")
    step = (64 << 20) // K
    for r0 in range(0, N, step):
        n = min(step, N - r0)
        w = synth.gaussian_torch(torch, 0x5EED0002, n * K, 0.0, 0.02, start=r0 * K).reshape(n, K)
        Q.encode_device(t, w, Wd[r0:r0 + n], n, K)
    x = synth.with_outliers(synth.gaussian(0x5EED1002, T * K), 0x5EED3002, 0.001, 20.0).reshape(T, K)
    q = quantized(Q, x)
    XR = q.max_k // K
    cap = torch.zeros(cap_ints(K, XR, N), dtype=torch.int32, device="cuda")
    y, y0 = run_dense(Q, t, Wd, q, N, K, T, XR, cap)
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32)), "the capture instantiation's outputs"
    del y, y0
    c = host(cap)
    del cap
    L = layout(K, XR)
    a = oracle.quantize_act(x, False)
    check_tokens(c, L, K, a["q"], a["d"], np.arange(T))
    W = host(Wd)
    for r0 in range(0, N, 4096):  # (the oracle's decode in slices: 4096 rows x 5120 floats at a time)
        rows = np.arange(r0, min(N, r0 + 4096))
        check_weights(oracle, t, W, K, c, L, N, rows)


@pytest.mark.parametrize("t,N,K", [(100, 768, 2048), (100, 2048, 768), (101, 300, 1024), (40, 512, 1024)])
def test_split_gemm_operands_expert_tiles(Q, oracle, t, N, K):
    """expert tiles (configs[3]'s gate / up and down shapes, and a partial row tile): the staged block of expert
    e's row r at w = e * N + r, the tokens by their input rows"""
    import torch
    E, n_used, T = 10, 4, 60
    L_ = Q.lib()
    W = oracle.quantize(t, synth.gaussian(310 + t, E * N * K, 0, 0.02).reshape(E * N, K))
    ids = (synth.splitmix64(311, T * n_used) % np.uint64(E)).astype(np.int32).reshape(T, n_used)
    tile = L_.qmatvec_id_batch_tile(t, N, K)
    assert tile == 64
    g = oracle.moe_group(ids, E, tile)
    x = synth.gaussian(312, T * K).reshape(T, K)
    q = quantized(Q, x)
    XR = q.max_k // K
    cap = torch.zeros(cap_ints(K, XR, E * N), dtype=torch.int32, device="cuda")
    y = torch.zeros((T * n_used, N), device="cuda")
    y0 = torch.zeros((T * n_used, N), device="cuda")
    bufs = [dev(np.array([g["n_tiles"]], np.int32)), dev(g["tile_e"]), dev(g["tile_start"]), dev(g["tile_n"]),
            dev(g["tok_rows"]), dev(g["pair_rows"])]
    Wd, rb = dev(W), Q.row_size(t, K)
    with Q.capture(cap):
        assert L_.qmatvec_launch_q8_id_batch(t, p(Wd), rb, q.ref, p(y), N, K, g["n_tiles"] + 2, tile,
                                             *[p(b) for b in bufs], None) == 0
    assert L_.qmatvec_launch_q8_id_batch(t, p(Wd), rb, q.ref, p(y0), N, K, g["n_tiles"] + 2, tile,
                                         *[p(b) for b in bufs], None) == 0
    a_, b_ = host(y), host(y0)
    assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32)), "the capture instantiation's outputs"
    c = host(cap)
    L = layout(K, XR)
    used = np.unique(ids)
    rows_seen = (used[:, None] * N + np.arange(N)[None, :]).reshape(-1)
    check_weights(oracle, t, W, K, c, L, E * N, rows_seen)
    a = oracle.quantize_act(x, False)
    check_tokens(c, L, K, a["q"], a["d"], np.unique(g["tok_rows"]))
