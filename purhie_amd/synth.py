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


def with_outliers(x, seed, frac=0.001, factor=20.0):
    """x with round(frac * size) entries at seeded distinct positions multiplied by factor"""
    x = np.array(x, dtype=np.float32, copy=True)
    flat = x.reshape(-1)
    k = int(round(frac * flat.size))
    u = uniform(seed, 4 * k + 16)
    pos = np.unique((u * flat.size).astype(np.int64).clip(0, flat.size - 1))[:k]
    flat[pos] *= np.float32(factor)
    return x


def seeds(cfg):
    return dict(w=0x5EED0000 + cfg, x=0x5EED1000 + cfg, router=0x5EED2000 + cfg, outlier=0x5EED3000 + cfg)
