import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def ref(oracle):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref/libref.so not built (needs the reference tree: make -f oracle/ref.mk)")
    return oracle


def pytest_terminal_summary(terminalreporter):
    """the per-output readings the fp32 parity checks recorded (tests/parity.py)"""
    try:
        from tests import parity
    except ImportError:
        return
    if not parity.STATS:
        return
    tr = terminalreporter
    tr.section("fp32 outputs: relative error and ULP distance (beside the 1e-5 * sum|w x| bound)")
    tr.write_line(f"{'category':58s} {'outputs':>9s} {'rel<=1e-5|<=2ulp':>17s} {'p99 rel':>9s} {'max rel':>9s} "
                  f"{'max ulp':>9s}")
    for k in sorted(parity.STATS):
        s = parity.STATS[k]
        frac = s["meet_rel1e-5_or_2ulp"] / max(s["outputs"], 1)
        tr.write_line(f"{k:58s} {s['outputs']:9d} {frac:17.6f} {s['p99_rel']:9.2e} {s['max_rel']:9.2e} "
                      f"{s['max_ulp']:9d}")
    path = os.environ.get("PURHIE_PARITY_STATS")
    if path:
        import json
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        with open(path, "w") as f:
            json.dump(parity.STATS, f, indent=1, sort_keys=True)
