"""The portable input generator (purhie_amd/synth.py): splitmix64 -> uniform -> Box-Muller in double -> float32.

gaussian_torch makes the benchmark's and the full-size tests' inputs on the device; these tests pin it to the
host generator gaussian() that the CPU path and the oracle use, and pin gaussian() itself to closed forms.
"""
import numpy as np
import pytest

from purhie_amd import synth


def test_splitmix64_known_outputs():
    # splitmix64 from state 0: the published first outputs of the generator (Vigna's reference implementation)
    got = synth.splitmix64(0, 3)
    assert [int(v) for v in got] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_uniform_and_box_muller_closed_forms():
    z = synth.splitmix64(11, 4)
    u = ((z >> np.uint64(11)).astype(np.float64) + 1.0) / 2.0 ** 53
    assert np.array_equal(synth.uniform(11, 4), u)
    assert (u > 0).all() and (u <= 1).all()
    g = synth.gaussian(11, 4).astype(np.float64)
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    want = np.array([r[0] * np.cos(2 * np.pi * u[1]), r[0] * np.sin(2 * np.pi * u[1]),
                     r[1] * np.cos(2 * np.pi * u[3]), r[1] * np.sin(2 * np.pi * u[3])]).astype(np.float32)
    assert np.array_equal(g.astype(np.float32), want)
    # moments of a large sample
    x = synth.gaussian(12, 1 << 20).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1.0) < 5e-3


def test_torch_generator_equals_host_on_cpu():
    torch = pytest.importorskip("torch")
    for seed, n, start, sd in ((0x5EED0001, 300001, 0, 0.02), (7, 200000, 1000, 1.0), (0x5EED2104, 65536, 0, 1.0)):
        want = synth.gaussian(seed, start + n, 0.0, sd)[start:]
        got = synth.gaussian_torch(torch, seed, n, 0.0, sd, start=start, device="cpu").numpy()
        assert np.array_equal(got, want), (seed, int((got != want).sum()))


def test_outlier_positions():
    pos = synth.outlier_positions(0x5EED3002, 2427 * 5120, 0.001)
    assert pos.size == round(0.001 * 2427 * 5120) and (np.diff(pos) > 0).all()
    x = synth.gaussian(3, 1000)
    y = synth.with_outliers(x, 5, 0.01, 20.0)
    p = synth.outlier_positions(5, 1000, 0.01)
    assert np.array_equal(y[p], x[p] * np.float32(20.0)) and np.array_equal(np.delete(y, p), np.delete(x, p))


@pytest.mark.gpu
def test_device_generator_equals_host():
    """the device's float64 log / sqrt / cos / sin may differ from the host's by an ulp; a float32 value differs
    only where that ulp crosses a float32 rounding boundary: at most a few in a billion. Exact here on the
    benchmark's MoE router logits (the routing the address replay in test_moe_prefill_bounds.py uses)."""
    import torch
    logits = synth.gaussian_torch(torch, 0x5EED2104, 512 * 128, 0.0, 1.0).cpu().numpy()
    assert np.array_equal(logits, synth.gaussian(0x5EED2104, 512 * 128))
    n, start = 4_000_000, 2_000_000
    want = synth.gaussian(0x5EED0003, start + n, 0.0, 0.02)[start:]
    got = synth.gaussian_torch(torch, 0x5EED0003, n, 0.0, 0.02, start=start).cpu().numpy()
    diff = got != want
    print(f"device generator: {int(diff.sum())} of {n} values differ from the host's", flush=True)
    assert diff.sum() <= 4
    if diff.any():
        ulps = np.abs(got.view(np.int32)[diff].astype(np.int64) - want.view(np.int32)[diff].astype(np.int64))
        assert ulps.max() <= 1
