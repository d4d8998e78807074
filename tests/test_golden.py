"""The golden vectors of tests/golden/ (written by tests/golden/make_golden.py from the reference's own CPU
code: quantize.cpp encoders, quant_types.cpp decoders, expert_cpu.cpp Q8_0 quantizer, matvec and expert FFN)
against the oracle (CPU) and against the HIP path (gpu)."""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = (8, 12, 13, 14, 23, 39, 40, 100, 101)
TOL = 1e-5


def load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


@pytest.mark.parametrize("t", TYPES)
def test_oracle_encoder_and_decoder_match_golden(oracle, t):
    g = load(f"enc_{t}.npz")
    b = oracle.quantize(t, g["x"])
    assert np.array_equal(b, g["bytes"])
    dec = oracle.to_float(t, g["bytes"], int(g["K"]))
    assert np.array_equal(dec.view(np.uint32), g["dec"].view(np.uint32))


def test_oracle_q8_0_activation_matches_golden(oracle):
    g = load("act_q8_0.npz")
    a = oracle.quantize_act(g["x"], kq=False)
    assert np.array_equal(a["q"], g["q"])
    assert np.array_equal(a["d"].view(np.uint32), g["d"].view(np.uint32))


@pytest.mark.parametrize("t", (8, 101))
def test_oracle_matvec_matches_golden(oracle, t):
    g = load(f"matvec_{t}.npz")
    N, K = int(g["N"]), int(g["K"])
    a = oracle.quantize_act(g["x"], kq=False)
    assert np.array_equal(a["q"], g["q"])
    want, _, mag = oracle.matvec(t, g["W"], N, K, a)
    assert np.all(np.abs(want - g["y"]) <= TOL * mag)


def test_oracle_expert_ffn_matches_golden(oracle):
    g = load("expert_ffn.npz")
    out = oracle.cpu_expert_ffn(g["gate"], g["up"], g["down"], int(g["FE"]), int(g["E"]), g["q"], g["d"])
    assert np.allclose(out, g["out"], rtol=1e-4, atol=1e-5 * np.abs(g["out"]).max())


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("t", TYPES)
def test_gpu_decoder_matches_golden(t):
    import torch
    from purhie_amd import qmatvec as Q
    g = load(f"enc_{t}.npz")
    n = g["dec"].size
    out = torch.zeros(n, dtype=torch.float32, device="cuda")
    Q.to_float_device(t, _dev(g["bytes"].reshape(-1)), out, n)
    assert np.array_equal(_host(out).view(np.uint32), g["dec"].reshape(-1).view(np.uint32))


@pytest.mark.gpu
def test_gpu_q8_0_activation_matches_golden():
    from purhie_amd import qmatvec as Q
    g = load("act_q8_0.npz")
    K = g["x"].size
    q = Q.Q8(K)
    Q.quantize(_dev(g["x"]), K, q)
    v = {k: _host(x) for k, x in q.views(K).items()}
    assert np.array_equal(v["q0"], g["q"])
    assert np.array_equal(v["d0"].view(np.uint32), g["d"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("t", (8, 101))
def test_gpu_matvec_matches_golden(oracle, t):
    """the HIP decode matvec against the reference CPU matvec's own output (expert_cpu.cpp)"""
    import torch
    from purhie_amd import qmatvec as Q
    g = load(f"matvec_{t}.npz")
    N, K = int(g["N"]), int(g["K"])
    q = Q.Q8(K)
    Q.quantize(_dev(g["x"]), K, q)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
    Q.launch_q8(t, _dev(g["W"]), q, y, N, K)
    _, _, mag = oracle.matvec(t, g["W"], N, K, oracle.quantize_act(g["x"], kq=False))
    assert np.all(np.abs(_host(y) - g["y"]) <= TOL * mag)
