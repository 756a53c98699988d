"""akh_sample_rows_noalloc: the sampler on the device's fixed workspace
(no allocation) against akh_sample_rows, through the C ABI.

Two calls in a row, the second smaller, each compared token for token with
akh_sample_rows on the same inputs (integer outputs: bit-exact), in greedy
and sampling modes; inside a captured graph on a fresh backend, where the
allocating akh_sample_rows is refused (its scratch cannot grow during
capture), replayed and compared with akh_sample_rows run outside capture;
and the workspace limit (rows * n <= 2^21) is enforced before anything runs.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(pkg, backend, rng, rows, n, ties=False):
    hip = pkg.hip
    l = (rng.standard_normal((rows, n)) * 2.5).astype(np.float32)
    if ties:
        l = np.round(l, 1).astype(np.float32)
    stride = 48
    seen = rng.integers(0, n, (rows, stride)).astype(np.uint32)
    lens = rng.integers(0, stride + 1, rows).astype(np.uint32)
    u = rng.random(rows)
    dev = dict(
        logits=hip.DeviceTensor(backend, l.nbytes).upload(l),
        seen=hip.DeviceTensor(backend, seen.nbytes).upload(seen),
        lens=hip.DeviceTensor(backend, lens.nbytes).upload(lens),
        u=hip.DeviceTensor(backend, u.nbytes).upload(u),
        out=hip.DeviceTensor(backend, rows * 4),
    )
    return dev, stride


def _both(backend, dev, stride, rows, n, t, k, p, pen):
    args = (dev["logits"], rows, n, dev["out"], t, k, p, pen, dev["seen"], stride,
            dev["lens"], dev["u"])
    backend.sample_rows_noalloc(*args)
    got = dev["out"].download(np.uint32, rows).copy()
    backend.sample_rows(*args)
    want = dev["out"].download(np.uint32, rows).copy()
    return got, want


def test_noalloc_sampler_matches_sample_rows(backend, pkg):
    rng = np.random.default_rng(77)
    # First call: 24 rows of the hall-1.0 vocabulary (1.2 M of the 2^21
    # workspace), run_chat's defaults (main.rs:162) and heavy ties.
    rows, n = 24, 50257
    dev, stride = _inputs(pkg, backend, rng, rows, n, ties=True)
    for t, k, p, pen in ((0.8, 40, 0.95, 1.15), (1.5, 0, 0.9, 1.0), (0.0, 0, 1.0, 1.3)):
        got, want = _both(backend, dev, stride, rows, n, t, k, p, pen)
        assert np.array_equal(got, want), (t, k, p, pen)
    # Second call, smaller: the workspace keeps the first call's contents,
    # which the sampler must not read.
    rows2, n2 = 5, 3001
    dev2, stride2 = _inputs(pkg, backend, rng, rows2, n2)
    for t, k, p, pen in ((1.0, 0, 1.0, 1.0), (0.5, 5, 1.0, 2.0), (0.0, 0, 1.0, 1.0)):
        got, want = _both(backend, dev2, stride2, rows2, n2, t, k, p, pen)
        assert np.array_equal(got, want), (t, k, p, pen)


def test_noalloc_sampler_inside_graph_capture(pkg):
    # The callers this entry point is for cannot allocate: here, code under
    # graph capture on a backend that has never grown its scratch.  Inputs
    # are allocated before the capture; the capture records the no-alloc
    # sampler, while akh_sample_rows is refused (its scratch would have to
    # grow).  Each replay, with eager work and a synchronisation between
    # replays, is checked against akh_sample_rows run outside capture.
    hip = pkg.hip
    be = hip.Backend(0)
    try:
        rng = np.random.default_rng(79)
        rows, n = 16, 50257
        dev, stride = _inputs(pkg, be, rng, rows, n, ties=True)
        params = (0.8, 40, 0.95, 1.15)
        args = (dev["logits"], rows, n, dev["out"], *params, dev["seen"], stride,
                dev["lens"], dev["u"])
        be.graph_begin()
        try:
            be.sample_rows_noalloc(*args)
            with pytest.raises(hip.InvalidArgument):
                be.sample_rows(*args)
        finally:
            g = be.graph_end()
        be.sample_rows(*args)  # eager, outside capture: grows the scratch
        want = dev["out"].download(np.uint32, rows).copy()
        for rep in range(3):
            dev["out"].upload(np.full(rows, 0xFFFFFFFF, np.uint32))
            g.execute()
            be.synchronize()
            got = dev["out"].download(np.uint32, rows).copy()
            assert np.array_equal(got, want), rep
            be.sample_rows(*args)  # eager work between the replays
            be.synchronize()
        g.close()
    finally:
        be.close()


def test_noalloc_sampler_rejects_oversized_input(backend, pkg):
    # 42 rows of 50257 ids need 2.11 M doubles, more than the 2^21 workspace:
    # rejected on the host before any launch.
    hip = pkg.hip
    rows, n = 42, 50257
    logits = hip.DeviceTensor(backend, 4)
    out = hip.DeviceTensor(backend, 4)
    with pytest.raises(hip.InvalidArgument):
        backend.sample_rows_noalloc(logits, rows, n, out, 0.0)
