"""Seeded synthetic inputs: splitmix64 -> uniform (0, 1] -> Box-Muller in double -> float32.

Portable by construction (no std::normal_distribution, whose output differs between standard
libraries). Per-config seeds: W 0x5EED0000 + cfg, x 0x5EED1000 + cfg, router 0x5EED2000 + cfg,
outliers 0x5EED3000 + cfg.
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, n):
    """n consecutive outputs of splitmix64 started at state `seed`"""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + _GOLDEN * np.arange(1, n + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed, n):
    """doubles in (0, 1]: the top 53 bits of each output, plus one, times 2^-53"""
    return ((splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def gaussian(seed, n, mean=0.0, sigma=1.0):
    """n float32 values ~N(mean, sigma^2), Box-Muller on consecutive pairs"""
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    th = 2.0 * np.pi * u[1::2]
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    return (mean + sigma * z[:n]).astype(np.float32)


def outlier_positions(seed, size, frac=0.001):
    """round(frac * size) seeded distinct positions in [0, size), ascending"""
    k = int(round(frac * size))
    u = uniform(seed, 4 * k + 16)
    return np.unique((u * size).astype(np.int64).clip(0, size - 1))[:k]


def with_outliers(x, seed, frac=0.001, factor=20.0):
    """x with round(frac * size) entries at seeded distinct positions multiplied by factor"""
    x = np.array(x, dtype=np.float32, copy=True)
    flat = x.reshape(-1)
    flat[outlier_positions(seed, flat.size, frac)] *= np.float32(factor)
    return x


def seeds(cfg):
    return dict(w=0x5EED0000 + cfg, x=0x5EED1000 + cfg, router=0x5EED2000 + cfg, outlier=0x5EED3000 + cfg)


def _i64(v):
    """a uint64 constant as the int64 of the same bits"""
    v = int(v)
    return v - (1 << 64) if v >= (1 << 63) else v


def gaussian_torch(torch, seed, n, mean=0.0, sigma=1.0, start=0, device="cuda"):
    """values start .. start + n - 1 (start even) of gaussian(seed, ...), made by torch on `device` (the benchmark's
    weights and activations, without a host round trip): the same splitmix64 outputs and uniforms bit for bit
    (int64 products wrap as the uint64 ones do; right shifts are masked to logical shifts), Box-Muller in float64
    with the device's log / sqrt / cos / sin, then float32. The float32 values equal gaussian()'s unless a device
    libm result differs from the host's by an ulp right at a float32 rounding boundary (a few in a billion)."""
    assert start % 2 == 0, "Box-Muller pairs start at even positions"
    m = (n + 1) // 2
    z = torch.arange(start + 1, start + 2 * m + 1, dtype=torch.int64, device=device) * _i64(_GOLDEN) + _i64(seed)
    z = (z ^ ((z >> 30) & ((1 << 34) - 1))) * _i64(_M1)
    z = (z ^ ((z >> 27) & ((1 << 37) - 1))) * _i64(_M2)
    z = z ^ ((z >> 31) & ((1 << 33) - 1))
    u = (((z >> 11) & ((1 << 53) - 1)).to(torch.float64) + 1.0) * (1.0 / 9007199254740992.0)
    del z
    r = torch.sqrt(-2.0 * torch.log(u[0::2]))
    th = 2.0 * np.pi * u[1::2]
    out = torch.empty(2 * m, dtype=torch.float64, device=device)
    out[0::2] = r * torch.cos(th)
    out[1::2] = r * torch.sin(th)
    return (mean + sigma * out[:n]).to(torch.float32)
