import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU")


def same_bits(got, want):
    """Bitwise equality of float32 arrays (NaN payloads compared by NaN-ness)."""
    g = np.ascontiguousarray(got, np.float32).reshape(-1)
    w = np.ascontiguousarray(want, np.float32).reshape(-1)
    assert g.shape == w.shape
    gn, wn = np.isnan(g), np.isnan(w)
    assert np.array_equal(gn, wn), "NaN positions differ"
    gb, wb = g.view(np.uint32)[~gn], w.view(np.uint32)[~wn]
    bad = np.nonzero(gb != wb)[0]
    assert bad.size == 0, "%d of %d differ; first at %d: got %r want %r" % (
        bad.size, gb.size, bad[0], g[~gn][bad[0]], w[~wn][bad[0]])


def rel_err(got, want):
    """The reference's per-element |a-b|/(1+|b|) (internal/compute/gpu/helpers_test.go:82)."""
    g = np.asarray(got, np.float64).reshape(-1)
    w = np.asarray(want, np.float64).reshape(-1)
    return float(np.max(np.abs(g - w) / (1.0 + np.abs(w)))) if g.size else 0.0


@pytest.fixture(scope="session")
def backend():
    from tcb_amd import QuantBackend
    b = QuantBackend(0)
    yield b
    b.close()


@pytest.fixture
def launch_shape(backend):
    """force(knob, a, b, c, d) forces a launch shape on the session context; every knob is reset afterwards."""
    used = []

    def force(knob, *vals):
        backend.ctx.set_launch_shape(knob, *vals)
        used.append(knob)

    yield force
    for k in used:
        backend.ctx.set_launch_shape(k)
