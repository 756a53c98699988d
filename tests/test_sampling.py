"""sample_token (src/nn/sampling.rs:3-81): the oracle restatement, and the
device sampler (akh_sample_rows) against it.

The reference draws r with rand::random(); here r is an input, so a draw
picks one token deterministically and the device must pick the same one as
the oracle.  The oracle is pinned by the reference's own tests
(sampling.rs:97-140) and by an independent vectorised numpy restatement.
"""

import numpy as np
import pytest

LOGITS = np.array([1.0, 4.0, 2.0, 8.0, 3.0], np.float32)  # sampling.rs:95


def _numpy_sample(logits, temperature, top_k, top_p, seen, penalty, r):
    """Vectorised restatement: stable argsort (ties lower index first),
    f64 probabilities, cumulative sums."""
    l = np.asarray(logits, np.float32).copy()
    if penalty != 1.0:
        for i in sorted(set(int(s) for s in seen)):
            if i < l.size:
                l[i] = np.float32(l[i] / np.float32(penalty)) if l[i] > 0 else np.float32(l[i] * np.float32(penalty))
    if temperature <= 0:
        return int(np.argmax(l))
    idx = np.argsort(-l.astype(np.float64), kind="stable")
    if 0 < top_k < idx.size:
        idx = idx[:top_k]
    p = np.exp((l[idx].astype(np.float64) - float(l[idx[0]])) / float(temperature))
    p = p / p.sum()
    if top_p < 1.0:
        c = np.cumsum(p)
        hit = np.nonzero(c >= np.float64(np.float32(top_p)))[0]
        keep = int(hit[0]) + 1 if hit.size else p.size
        idx, p = idx[:keep], p[:keep]
        p = p / p.sum()
    c = np.cumsum(p)
    hit = np.nonzero(r < c)[0]
    return int(idx[hit[0]]) if hit.size else int(idx[-1])


# ---- the oracle ----------------------------------------------------------

def test_reference_sampling_tests_on_oracle(ora):
    rng = np.random.default_rng(0)
    for r in rng.random(20):
        assert ora.sample_token(LOGITS, 0.0, 0, 1.0, [], 1.0, r) == 3      # zero_temperature_is_greedy
        assert ora.sample_token(LOGITS, 1.5, 1, 1.0, [], 1.0, r) == 3      # top_k_one_is_greedy
        assert ora.sample_token(LOGITS, 1.0, 0, 0.01, [], 1.0, r) == 3     # tiny_top_p_is_greedy
    for r in rng.random(50):
        assert ora.sample_token(LOGITS, 2.0, 2, 1.0, [], 1.0, r) in (1, 3)  # top_k_restricts
    seen = {ora.sample_token(LOGITS, 100.0, 0, 1.0, [], 1.0, r) for r in rng.random(2000)}
    assert seen == {0, 1, 2, 3, 4}                                         # filters_off_can_reach_every_token
    assert ora.sample_token(LOGITS, 0.0, 0, 1.0, [], 1.0, 0.3) == 3        # repetition_penalty_demotes...
    assert ora.sample_token(LOGITS, 0.0, 0, 1.0, [3], 100.0, 0.3) == 1


def test_oracle_matches_vectorised_restatement(ora):
    rng = np.random.default_rng(1)
    cases = [(0.8, 40, 0.95, 1.15), (1.0, 0, 1.0, 1.0), (1.5, 0, 0.9, 1.0),
             (0.5, 5, 1.0, 2.0), (0.0, 0, 1.0, 1.3), (2.0, 300, 0.5, 1.0)]
    for t, k, p, pen in cases:
        for _ in range(12):
            n = int(rng.integers(50, 3000))
            l = (rng.standard_normal(n) * 3).astype(np.float32)
            if rng.random() < 0.3:
                l = np.round(l, 1).astype(np.float32)  # many ties
            seen = rng.integers(0, n, int(rng.integers(0, 40))).astype(np.uint32)
            r = float(rng.random())
            assert ora.sample_token(l, t, k, p, seen, pen, r) == _numpy_sample(l, t, k, p, seen, pen, r)


# ---- the device sampler --------------------------------------------------

def _device_sample(pkg, backend, logits, t, k, p, pen, seen_rows, uniforms):
    hip = pkg.hip
    rows, n = logits.shape
    dl = hip.DeviceTensor(backend, logits.nbytes).upload(np.ascontiguousarray(logits))
    stride = max(1, max(len(s) for s in seen_rows))
    seen = np.zeros((rows, stride), np.uint32)
    lens = np.zeros(rows, np.uint32)
    for i, s in enumerate(seen_rows):
        seen[i, :len(s)] = s
        lens[i] = len(s)
    ds = hip.DeviceTensor(backend, seen.nbytes).upload(seen)
    dn = hip.DeviceTensor(backend, lens.nbytes).upload(lens)
    du = hip.DeviceTensor(backend, uniforms.nbytes).upload(uniforms.astype(np.float64))
    do = hip.DeviceTensor(backend, rows * 4)
    backend.sample_rows(dl, rows, n, do, t, k, p, pen, ds, stride, dn, du)
    return do.download(np.uint32, rows)


@pytest.mark.gpu
def test_device_reference_tests(backend, pkg):
    rng = np.random.default_rng(2)
    u = rng.random(20)
    l = np.tile(LOGITS, (20, 1))
    none = [[]] * 20
    assert list(_device_sample(pkg, backend, l, 0.0, 0, 1.0, 1.0, none, u)) == [3] * 20
    assert list(_device_sample(pkg, backend, l, 1.5, 1, 1.0, 1.0, none, u)) == [3] * 20
    assert list(_device_sample(pkg, backend, l, 1.0, 0, 0.01, 1.0, none, u)) == [3] * 20
    assert set(_device_sample(pkg, backend, l, 2.0, 2, 1.0, 1.0, none, u)) <= {1, 3}
    ll = np.tile(LOGITS, (500, 1))
    got = _device_sample(pkg, backend, ll, 100.0, 0, 1.0, 1.0, [[]] * 500, rng.random(500))
    assert set(got) == {0, 1, 2, 3, 4}
    assert list(_device_sample(pkg, backend, l[:1], 0.0, 0, 1.0, 100.0, [[3]], u[:1])) == [1]
    # Greedy over NaN logits follows the reference's scan from index 0: a NaN
    # at index 0 stays the answer, a NaN elsewhere never wins.
    nanl = np.tile(LOGITS, (2, 1))
    nanl[0, 0] = np.nan
    nanl[1, 2] = np.nan
    assert list(_device_sample(pkg, backend, nanl, 0.0, 0, 1.0, 1.0, [[]] * 2, u[:2])) == [0, 3]


@pytest.mark.gpu
@pytest.mark.parametrize("t,k,p,pen,ties", [
    (0.8, 40, 0.95, 1.15, False),  # run_chat's defaults (main.rs:162)
    (1.0, 0, 1.0, 1.0, False),
    (1.5, 0, 0.9, 1.0, False),
    (0.5, 5, 1.0, 2.0, False),
    (0.0, 0, 1.0, 1.3, False),
    (1.0, 100, 0.9, 1.0, True),
    (3.0, 0, 0.999, 1.05, True),
])
def test_device_sampler_matches_oracle(backend, pkg, ora, t, k, p, pen, ties):
    rng = np.random.default_rng(int(t * 10 + k + p * 100))
    rows, n = 16, 50257
    l = (rng.standard_normal((rows, n)) * 2.5).astype(np.float32)
    if ties:
        l = np.round(l, 1).astype(np.float32)
    seen_rows = [rng.integers(0, n, int(rng.integers(0, 64))).astype(np.uint32) for _ in range(rows)]
    u = rng.random(rows)
    got = _device_sample(pkg, backend, l, t, k, p, pen, seen_rows, u)
    want = [ora.sample_token(l[i], t, k, p, seen_rows[i], pen, u[i]) for i in range(rows)]
    assert list(got) == want


@pytest.mark.gpu
@pytest.mark.parametrize("rows,k", [(4, 40), (64, 40), (3, 200)])
def test_device_sampler_split_rows_edge_cases(backend, pkg, ora, rows, k):
    # run_chat's parameters with rows split over parts of the vocabulary (16
    # parts at 4 rows, 4 at 64; top_k 200 at 3 rows: 10 parts, so that all
    # parts' top_k fit the merge): a quarter of the vocabulary at -inf (parts
    # with no finite element), only 10 finite logits (fewer than top_k: the
    # radix path), integer logits (ties across parts, lower index first),
    # and plain rows; every row against the oracle.
    rng = np.random.default_rng(77 + rows)
    n = 50257
    l = (rng.standard_normal((rows, n)) * 2.5).astype(np.float32)
    l[0, : n // 4] = -np.inf
    l[1, :] = -np.inf
    l[1, rng.choice(n, 10, replace=False)] = rng.standard_normal(10).astype(np.float32)
    l[2] = np.round(l[2]).astype(np.float32)
    seen_rows = [rng.integers(0, n, int(rng.integers(0, 64))).astype(np.uint32) for _ in range(rows)]
    u = rng.random(rows)
    got = _device_sample(pkg, backend, l, 0.8, k, 0.95, 1.15, seen_rows, u)
    want = [ora.sample_token(l[i], 0.8, k, 0.95, seen_rows[i], 1.15, u[i]) for i in range(rows)]
    assert list(got) == want
