"""fp32 output checks shared by the GPU parity tests.

Each check asserts the reference's own bound, |y - y_ref| <= 1e-5 * sum |w x| (tests/matvec_verify.cpp:8,142),
and records the per-output reading beside it: the relative error |y - y_ref| / |y_ref| and the fp32 ULP distance,
and whether each output meets "relative error <= 1e-5 or <= 2 ULP". The records are summed per category and
printed at the end of the session (tests/conftest.py); with PURHIE_PARITY_STATS=<path> they are also written there
as JSON. y_ref is the oracle's fp32 sum in the reference CPU path's order ("cpu") or the double sum of decoded
weights times decoded activations ("f64").
"""
import numpy as np

STATS = {}


def ulp_distance(a, b):
    """distance of fp32 values in units in the last place (ordered bit patterns; +0 and -0 are 0 apart)"""
    def line(x):
        i = np.asarray(x, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(line(a) - line(b))


def record(name, got, want):
    """adds the per-output relative error and ULP distance of got against want to category `name`"""
    got = np.asarray(got, np.float32).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = np.abs(got.astype(np.float64) - want)
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.where(err == 0, 0.0, err / np.abs(want))
    ulp = ulp_distance(got, want.astype(np.float32))
    meets = (rel <= 1e-5) | (ulp <= 2)
    s = STATS.setdefault(name, {"outputs": 0, "meet_rel1e-5_or_2ulp": 0, "max_rel": 0.0, "max_ulp": 0,
                                "p99_rel": 0.0})
    s["outputs"] += int(got.size)
    s["meet_rel1e-5_or_2ulp"] += int(meets.sum())
    finite = rel[np.isfinite(rel)]
    if finite.size:
        s["max_rel"] = max(s["max_rel"], float(finite.max()))
        s["p99_rel"] = max(s["p99_rel"], float(np.quantile(finite, 0.99)))
    s["max_ulp"] = max(s["max_ulp"], int(ulp.max()) if ulp.size else 0)


def check(name, got, want, mag, ref=None, tol=1e-5):
    """asserts |got - want| <= tol * mag (and the same against ref when given) and records both readings"""
    got = np.asarray(got, np.float32)
    want = np.asarray(want)
    mag = np.asarray(mag, np.float64)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    worst = float((err / (mag + 1e-30)).max()) if err.size else 0.0
    assert np.all(err <= tol * mag), f"{name}: max |y - y_cpu| / sum|w x| = {worst:.3g} > {tol}"
    record(name + " vs cpu", got, want)
    if ref is not None:
        e2 = np.abs(got.astype(np.float64) - np.asarray(ref, np.float64))
        assert np.all(e2 <= tol * mag), f"{name}: max |y - y_f64| / sum|w x| = {float((e2 / (mag + 1e-30)).max()):.3g}"
        record(name + " vs f64", got, ref)
