"""Per-shader launchers of libakasha_hip.so against the CPU oracle.

Shapes, seeds and tolerances follow the reference's own kernel tests
(src/nn/ops/emit.rs:1001-1503) where they exist.  Every call goes through
the C ABI on the GPU.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _meta(be, m):
    return be.meta(m)


def test_embedding(backend, pkg, ora):
    h = pkg.hip
    vocab, dim = 11, 300
    table = ora.rand_vec(vocab * dim, 3)
    toks = np.array([0, 10, 11, 5, 4294967295, 3], np.uint32)
    out = backend.zeros(len(toks) * dim)
    shape = h.EmbeddingMeta(vocab, dim, len(toks))
    backend.embedding(backend.tensor(toks), backend.tensor(table), out, shape, _meta(backend, shape))
    got = out.download()
    assert np.array_equal(got, ora.embedding(toks, table, vocab, dim, len(toks)))


def test_tensor_reuse_is_ordered_on_the_stream(backend):
    # A freed tensor's block is handed out again without waiting for the
    # stream: the new tensor's zeroing is queued behind the kernels still
    # writing the old one.
    n = 1 << 24
    old = backend.tensor(np.full(n, 2.0, np.float32))
    addr = old.ptr.value
    for _ in range(20):
        backend.silu(old, n)
    old.free()
    new = backend.zeros(n)
    assert new.ptr.value == addr
    assert not new.download().any()
    new.free()


def test_tensor_double_free_is_refused(backend, pkg):
    # A freed block waits in the backend's pool: freeing it again is an
    # error, not a second hipFree of memory a later alloc may hand out.
    h = pkg.hip
    t = backend.zeros(1000)
    p = t.ptr
    t.free()
    assert h._lib.akh_tensor_free(backend.handle, p) == h.InvalidArgument.code
    assert b"already freed" in h._lib.akh_last_error()
    again = backend.zeros(1000)
    assert again.ptr.value == p.value and not again.download().any()
    again.free()


def test_tensor_pool_random_reuse(backend):
    # Seeded random allocations, uploads, frees and queued kernels on one
    # backend: every new tensor reads zero, every live tensor keeps what was
    # last written to it, whichever pooled block it landed on.
    rng = np.random.default_rng(5)
    live = []
    for _ in range(300):
        op = rng.random()
        if op < 0.45 or not live:
            n = int(rng.choice([1, 7, 1000, 4096, 65537, 300000]))
            t = backend.zeros(n)
            assert not t.download()[:n].any()
            v = rng.standard_normal(n).astype(np.float32)
            if rng.random() < 0.5:
                t.upload(v)
            else:
                v = np.zeros(n, np.float32)
            live.append((t, v))
        elif op < 0.8:
            t, v = live.pop(int(rng.integers(len(live))))
            assert np.array_equal(t.download()[: v.size], v)
            t.free()
        else:
            t, v = live[int(rng.integers(len(live)))]
            backend.silu(t, v.size)  # queued work on a live tensor
            v[:] = v / (np.float32(1) + np.exp(-v))
            np.testing.assert_allclose(t.download()[: v.size], v, rtol=2e-6, atol=1e-7)
            live[[x[0] for x in live].index(t)] = (t, t.download()[: v.size].copy())
    for t, v in live:
        assert np.array_equal(t.download()[: v.size], v)
        t.free()


def test_tensor_from_host(backend, pkg):
    # Tensor::init_from_cpu in one call (no zero fill): the copy is taken
    # before the call returns, small (staged) and large alike.
    h = pkg.hip
    for n in (1, 3, 1000, 16384, 300000):
        a = np.arange(n, dtype=np.float32) - 7.5
        host = a.copy()
        t = backend.tensor(host)
        host[:] = 3.0
        assert np.array_equal(t.download()[:n], a)
        t.free()
    m = h.MatMulMeta(5, 6, 7)
    t = backend.meta(m)
    assert list(t.download(np.uint32, 3)) == [5, 6, 7]
    t.free()


def test_uploads_are_staged_and_ordered(backend):
    # Uploads return before the copy runs: the host array is copied out at
    # once (changing it afterwards changes nothing), a kernel queued after an
    # upload sees the data, and more uploads than staging slots all land.
    a = np.linspace(-4, 4, 5000, dtype=np.float32)
    t = backend.zeros(a.size)
    host = a.copy()
    t.upload(host)
    host[:] = 7.0
    backend.silu(t, a.size)
    exp = a / (np.float32(1) + np.exp(-a))
    np.testing.assert_allclose(t.download(), exp, rtol=2e-6, atol=1e-7)
    rng = np.random.default_rng(3)
    datas = [rng.standard_normal(1000 + 37 * i).astype(np.float32) for i in range(150)]
    ts = [backend.zeros(d.size) for d in datas]
    for x, d in zip(ts, datas):
        x.upload(d)
    for x, d in zip(ts, datas):
        assert np.array_equal(x.download(), d)
    big = rng.standard_normal(1 << 20).astype(np.float32)  # past one staging slot
    tb = backend.zeros(big.size)
    tb.upload(big)
    assert np.array_equal(tb.download(), big)


@pytest.mark.parametrize("rows,size", [(5, 96), (3, 768), (1, 32)])
def test_rmsnorm(backend, pkg, ora, rows, size):
    h = pkg.hip
    x = ora.rand_vec(rows * size, 9) * 3
    w = 1 + ora.rand_vec(size, 10) * 0.1
    out = backend.zeros(rows * size)
    shape = h.NormMeta(rows, size, 1e-5)
    backend.rmsnorm(backend.tensor(x), backend.tensor(w), out, shape, _meta(backend, shape))
    np.testing.assert_allclose(out.download(), ora.rmsnorm(x, w, rows, size, 1e-5),
                               rtol=1e-5, atol=1e-6)


def test_gemv_routing(backend, pkg, ora):
    # gemv_routing_matches_cpu_reference (emit.rs:1424-1465): n=301, k=19.
    h = pkg.hip
    n, k = 301, 19
    a, b, c0 = ora.rand_vec(k, 10), ora.rand_vec(k * n, 20), ora.rand_vec(n, 30)
    shape = h.MatMulMeta(1, n, k)
    meta = _meta(backend, shape)
    c = backend.zeros(n)
    cadd = backend.tensor(c0)
    ta, tb = backend.tensor(a), backend.tensor(b)
    backend.matmul(ta, tb, c, shape, meta)
    backend.matmul_add(ta, tb, cadd, shape, meta)
    assert np.abs(c.download() - ora.matmul(a, b, 1, n, k)).max() < 1e-4
    assert np.abs(cadd.download() - ora.matmul_add(a, b, c0, 1, n, k)).max() < 1e-4


@pytest.mark.parametrize("m,n,k", [(37, 301, 19), (2, 50257, 768), (32, 768, 3072),
                                   (128, 128, 64), (200, 2304, 768), (513, 130, 37),
                                   # small m: K split over the part (decode's GEMVs)
                                   (1, 768, 3072), (1, 2304, 768), (5, 3072, 768), (1, 3, 5),
                                   (1, 1000, 1), (17, 768, 768),
                                   # rows not whole 16-byte pieces: lane-adjacent columns
                                   (1, 50257, 768), (4, 1001, 513),
                                   # prompt-sized m: K split where the tiles are few
                                   (64, 768, 3072), (64, 2304, 768), (512, 768, 3072)])
def test_matmul_and_add(backend, pkg, ora, m, n, k):
    h = pkg.hip
    a, b = ora.rand_vec(m * k, 1), ora.rand_vec(k * n, 2)
    c0 = ora.rand_vec(m * n, 3)
    shape = h.MatMulMeta(m, n, k)
    meta = _meta(backend, shape)
    ta, tb = backend.tensor(a), backend.tensor(b)
    c, cadd = backend.zeros(m * n), backend.tensor(c0)
    backend.matmul(ta, tb, c, shape, meta)
    backend.matmul_add(ta, tb, cadd, shape, meta)
    ref = ora.matmul(a, b, m, n, k)
    tol = 1e-4 * max(1.0, np.sqrt(k / 19.0))
    assert np.abs(c.download() - ref).max() < tol
    assert np.abs(cadd.download() - ora.matmul_add(a, b, c0, m, n, k)).max() < tol


def test_matmul_live_meta_bounds_work(backend, pkg, ora):
    # Grid sized for the build-time shape; the live meta shrinks m and n.
    h = pkg.hip
    M, N, K = 64, 256, 32
    a, b = ora.rand_vec(M * K, 4), ora.rand_vec(K * N, 5)
    sentinel = np.full(M * N, 7.0, np.float32)
    for m, n in ((40, 200), (1, 100)):
        c = backend.tensor(sentinel)
        live = h.MatMulMeta(m, n, K)
        backend.matmul(backend.tensor(a), backend.tensor(b[: K * n].copy()), c,
                       h.MatMulMeta(M, N, K), _meta(backend, live))
        got = c.download()
        ref = ora.matmul(a[: m * K], b[: K * n], m, n, K)
        assert np.abs(got[: m * n] - ref).max() < 1e-4
        assert np.all(got[m * n:] == 7.0)


@pytest.mark.parametrize("M,K,N", [(4, 768, 2304), (1, 768, 2304), (1, 3072, 2304), (1, 768, 2305)])
def test_small_m_matmul_k_split_live_meta(backend, pkg, ora, M, K, N):
    # Small-m MATMUL splits K over blocks whose partial sums the last block
    # of each column slab adds.  The grid and splits follow the recorded
    # shape; live metas shrink m, n and k, so some splits get no rows and
    # some slabs no columns (they must neither count nor store).  Every call
    # after the first reuses the workspace and its counters; the same call
    # twice gives the same bits.
    # With M = 1 the recorded shape runs 1024-thread blocks over ranges of
    # 768 rows of K: one range (K = 768, no partial sums) or four; N = 2305
    # (rows not whole 16-byte pieces) takes lane-adjacent columns.
    h = pkg.hip
    a, b = ora.rand_vec(M * K, 11), ora.rand_vec(K * N, 12)
    c0 = ora.rand_vec(M * N, 13)
    rec = h.MatMulMeta(M, N, K)
    live = ((4, 2304, 768), (1, 2304, 768), (3, 1000, 300), (2, 257, 7), (4, 2304, 768))
    for m, n, k in ((min(m, M), n, k) for m, n, k in live):
        tb = backend.tensor(b[: k * n].copy())
        am = a.reshape(M, K)[:m, :k].copy().ravel()
        tam = backend.tensor(am)
        meta = _meta(backend, h.MatMulMeta(m, n, k))
        outs = []
        for _ in range(2):
            c = backend.tensor(np.full(M * N, 7.0, np.float32))
            backend.matmul(tam, tb, c, rec, meta)
            outs.append(c.download())
        cadd = backend.tensor(c0)
        backend.matmul_add(tam, tb, cadd, rec, meta)
        ref = ora.matmul(am, b[: k * n], m, n, k)
        tol = 1e-4 * max(1.0, np.sqrt(k / 19.0))
        assert np.abs(outs[0][: m * n] - ref).max() < tol, (m, n, k)
        assert np.all(outs[0][m * n:] == 7.0)
        assert np.array_equal(outs[0], outs[1])
        got = cadd.download()
        assert np.abs(got[: m * n] - ora.matmul_add(am, b[: k * n], c0[: m * n], m, n, k)).max() < tol
        assert np.array_equal(got[m * n:], c0[m * n:])


def test_prompt_m_matmul_k_split_live_meta(backend, pkg, ora):
    # m > 32 on a grid of fewer tiles than CUs splits K over several blocks
    # per tile, whose partial sums the tile's last block adds.  Live metas
    # shrink m, n and k under the recorded shape's grid and splits, so some
    # splits get no rows and some tiles no rows or columns; repeated calls
    # reuse the workspace and counters and give the same bits.
    h = pkg.hip
    M, N, K = 100, 768, 3072
    a, b = ora.rand_vec(M * K, 21), ora.rand_vec(K * N, 22)
    c0 = ora.rand_vec(M * N, 23)
    rec = h.MatMulMeta(M, N, K)
    for m, n, k in ((100, 768, 3072), (70, 500, 1000), (33, 129, 40), (100, 768, 3072)):
        am = a.reshape(M, K)[:m, :k].copy().ravel()
        tam, tb = backend.tensor(am), backend.tensor(b[: k * n].copy())
        meta = _meta(backend, h.MatMulMeta(m, n, k))
        outs = []
        for _ in range(2):
            c = backend.tensor(np.full(M * N, 7.0, np.float32))
            backend.matmul(tam, tb, c, rec, meta)
            outs.append(c.download())
        cadd = backend.tensor(c0)
        backend.matmul_add(tam, tb, cadd, rec, meta)
        ref = ora.matmul(am, b[: k * n], m, n, k)
        tol = 1e-4 * max(1.0, np.sqrt(k / 19.0))
        assert np.abs(outs[0][: m * n] - ref).max() < tol, (m, n, k)
        assert np.all(outs[0][m * n:] == 7.0)
        assert np.array_equal(outs[0], outs[1])
        got = cadd.download()
        assert np.abs(got[: m * n] - ora.matmul_add(am, b[: k * n], c0[: m * n], m, n, k)).max() < tol
        assert np.array_equal(got[m * n:], c0[m * n:])


@pytest.mark.parametrize("M,K,N", [(1, 768, 2304), (1, 3072, 768), (4, 768, 2304),
                                   (1, 768, 2305), (100, 3072, 768), (2048, 64, 2048)])
def test_matmul_live_meta_beyond_recorded_is_clamped(backend, pkg, ora, M, K, N):
    # A live meta larger than the recorded shape in m, n and k computes the
    # recorded product and writes nothing past it.  The operands carry extra
    # data after the recorded extent (so a read past it would change the
    # sums, not leave the buffers); C's tail keeps its sentinel.  Shapes: the
    # m = 1 GEMV over one range of K and over four, the m = 4 GEMV, the
    # lane-adjacent-column GEMV, the K-split MFMA GEMM and the unsplit one
    # (256 tiles).
    h = pkg.hip
    pad = 4096
    a, b = ora.rand_vec(M * K + pad, 31), ora.rand_vec(K * N + pad, 32)
    c0 = ora.rand_vec(M * N + pad, 33)
    rec = h.MatMulMeta(M, N, K)
    meta = _meta(backend, h.MatMulMeta(M + 3, N + 5, K + 7))
    ta, tb = backend.tensor(a), backend.tensor(b)
    c = backend.tensor(np.full(M * N + pad, 7.0, np.float32))
    backend.matmul(ta, tb, c, rec, meta)
    cadd = backend.tensor(c0)
    backend.matmul_add(ta, tb, cadd, rec, meta)
    tol = 1e-4 * max(1.0, np.sqrt(K / 19.0))
    got = c.download()
    assert np.abs(got[: M * N] - ora.matmul(a[: M * K], b[: K * N], M, N, K)).max() < tol
    assert np.all(got[M * N:] == 7.0)
    got = cadd.download()
    ref = ora.matmul_add(a[: M * K], b[: K * N], c0[: M * N], M, N, K)
    assert np.abs(got[: M * N] - ref).max() < tol
    assert np.array_equal(got[M * N:], c0[M * N:])


@pytest.mark.parametrize("seq,dim", [(8, 4), (37, 12), (65, 48)])
def test_head_gather_qkv_slices(backend, pkg, ora, seq, dim):
    # qkv_split_matches_three_head_gathers shapes (emit.rs:1227-1231).
    h = pkg.hip
    src = ora.rand_vec(seq * 3 * dim, 50)
    t = backend.tensor(src)
    for role in range(3):
        out = backend.zeros(seq * dim)
        shape = h.HeadMoveMeta(seq, 3 * dim, dim, role * dim)
        backend.head_gather(t, out, shape, _meta(backend, shape))
        assert np.array_equal(out.download(), ora.head_gather(src, seq, 3 * dim, dim, role * dim))


@pytest.mark.parametrize("seq,dim,hd", [(8, 8, 4), (37, 12, 4), (65, 48, 16)])
def test_rope_and_offset(backend, pkg, ora, seq, dim, hd):
    h = pkg.hip
    x = ora.rand_vec(seq * dim, 10)
    buf = backend.tensor(x)
    shape = h.RopeMeta(seq, dim, hd, 0)
    backend.rope(buf, shape, _meta(backend, shape))
    assert np.abs(buf.download() - ora.rope(x, seq, dim, hd)).max() < 1e-4
    for pos in (0, 5, 511):
        row = x[:dim].copy()
        rb = backend.tensor(row)
        s2 = h.RopeOffsetMeta(1, dim, hd, pos)
        backend.rope_offset(rb, s2, _meta(backend, s2))
        assert np.abs(rb.download() - ora.rope_offset(row, 1, dim, hd, pos)).max() < 1e-4


def test_cache_write(backend, pkg, ora):
    h = pkg.hip
    src, dst = ora.rand_vec(3 * 64, 1), ora.rand_vec(10 * 64, 2)
    t = backend.tensor(dst)
    shape = h.CacheWriteMeta(3, 64, 4)
    backend.cache_write(backend.tensor(src), t, shape, _meta(backend, shape))
    assert np.array_equal(t.download(), ora.cache_write(src, dst, 3, 64, 4))


def _flash(backend, h, q, k, v, seq, dim, hd, row_offset=0, total_rows=None):
    total_rows = total_rows or seq
    out = backend.zeros(total_rows * dim)
    lse = backend.zeros(seq * (dim // hd))
    shape = h.FlashAttnMeta(seq, dim, hd, np.float32(1.0) / np.sqrt(np.float32(hd)), row_offset)
    backend.flash_attention(backend.tensor(q), backend.tensor(k), backend.tensor(v), out, lse,
                            shape, _meta(backend, shape))
    return out.download(), lse.download()


@pytest.mark.parametrize("seq,heads,hd", [(8, 2, 4), (37, 3, 16), (65, 12, 64), (200, 2, 64),
                                          (130, 1, 128), (300, 2, 128), (1024, 4, 128),
                                          # head sizes that are not powers of two (emit.rs:
                                          # 564-572 takes any head_dim <= 128)
                                          (40, 2, 6), (33, 3, 12), (50, 4, 24), (77, 2, 48),
                                          (200, 2, 80), (130, 3, 96), (150, 1, 100),
                                          # head sizes that are not multiples of 4: rows
                                          # without 16-byte alignment, loaded element by
                                          # element
                                          (70, 2, 34), (90, 3, 50), (140, 2, 126), (60, 3, 33),
                                          (45, 1, 65)])
def test_flash_attention(backend, pkg, ora, seq, heads, hd):
    # flash_attention_matches_cpu_reference (emit.rs:1001-1098), tol 1e-3.
    h = pkg.hip
    dim = heads * hd
    n = seq * dim
    q, k, v = ora.rand_vec(n, 1), ora.rand_vec(n, 2), ora.rand_vec(n, 3)
    got, lse = _flash(backend, h, q, k, v, seq, dim, hd)
    ref = ora.causal_attention(q, k, v, seq, dim, hd)
    assert np.abs(got - ref).max() < 1e-3
    # l_cache = max + ln(sum) of the scaled scores (cuda.rs:680-682).
    Q, K = q.reshape(seq, dim).astype(np.float64), k.reshape(seq, dim).astype(np.float64)
    V = v.reshape(seq, dim).astype(np.float64)
    for hh in range(heads):
        sl = slice(hh * hd, (hh + 1) * hd)
        s = Q[:, sl] @ K[:, sl].T / np.sqrt(hd)
        s[np.triu_indices(seq, 1)] = -np.inf
        ref_l = np.log(np.exp(s - s.max(1, keepdims=True)).sum(1)) + s.max(1)
        assert np.abs(lse.reshape(seq, heads)[:, hh] - ref_l).max() < 1e-3
        if hd > 32:
            # Head sizes above 32 run on split-bfloat16 MFMAs: fp32-level
            # error against a float64 reference (the fp32-MFMA kernel's is
            # ~1e-6).
            w = np.exp(s - s.max(1, keepdims=True))
            ref64 = (w / w.sum(1, keepdims=True)) @ V[:, sl]
            assert np.abs(got.reshape(seq, dim)[:, sl] - ref64).max() < 1e-5
            assert np.abs(lse.reshape(seq, heads)[:, hh] - ref_l).max() < 1e-5


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("where", ["none", "q", "k", "v"])
def test_flash_attention_beyond_fp16_range(backend, pkg, ora, hd, where):
    # A small grid runs split-fp16 tiles; a tile with an operand beyond
    # fp16's range (|x| >= 65520) recomputes itself on split-bf16 products,
    # so every tile matches a float64 reference to fp32 level.  The large
    # entry's partner dims are scaled down so the scores stay moderate (an
    # fp32 score of 1e4 would already move the weights by ~1e-3).
    h = pkg.hip
    heads, S = 2, 160
    dim = heads * hd
    q, k, v = (ora.rand_vec(S * dim, 60 + i).reshape(S, dim) for i in range(3))
    if where == "q":
        q[100, 5] = 1.0e5
        k[:, 5] *= 1e-4
    elif where == "k":
        k[37, hd + 3] = -7.0e4
        q[:, hd + 3] *= 1e-4
    elif where == "v":
        v[50, 7] = 9.0e4
    got, lse = _flash(backend, h, q.ravel(), k.ravel(), v.ravel(), S, dim, hd)
    got = got.reshape(S, dim)
    Q, K, V = (x.astype(np.float64) for x in (q, k, v))
    for hh in range(heads):
        sl = slice(hh * hd, (hh + 1) * hd)
        s = Q[:, sl] @ K[:, sl].T / np.sqrt(hd)
        s[np.triu_indices(S, 1)] = -np.inf
        w = np.exp(s - s.max(1, keepdims=True))
        ref = (w / w.sum(1, keepdims=True)) @ V[:, sl]
        tol = 1e-5 * (1.0 + np.abs(V[:, sl]).max(0))
        assert np.all(np.abs(got[:, sl] - ref) <= tol), (where, hh)
        ref_l = np.log(w.sum(1)) + s.max(1)
        assert np.abs(lse.reshape(S, heads)[:, hh] - ref_l).max() < 1e-5


def test_flash_attention_batched_beyond_fp16_range(backend, pkg):
    # A grid of 128-query tiles as large as the part (8 x 8 x 4 = 256 blocks)
    # runs split-fp16 tiles that recompute themselves on split-bf16 products
    # when an operand is beyond fp16's range: sequence 3 holds such a K entry
    # and sequence 6 such a V entry; sequence 0 has none.  Each matches a
    # float64 reference to fp32 level.
    h = pkg.hip
    B, S, H, hd = 8, 512, 8, 64
    d = H * hd
    rng = np.random.default_rng(70)
    q, k, v = (rng.standard_normal((B, S, d), dtype=np.float32) for _ in range(3))
    k[3, 100, 5] = 7.0e4
    q[3, :, 5] *= 1e-4
    v[6, 200, hd + 6] = -9.0e4
    out, lse = backend.zeros(B * S * d), backend.zeros(B * S * H)
    shape = h.FlashAttnMeta(S, d, hd, 0.125, 0)
    backend.flash_attention_batched(backend.tensor(q.ravel()), backend.tensor(k.ravel()),
                                    backend.tensor(v.ravel()), out, lse, shape,
                                    _meta(backend, shape), B)
    got = out.download().reshape(B, S, d)
    for b in (0, 3, 6):
        Q, K, V = (x[b].astype(np.float64) for x in (q, k, v))
        for hh in (0, 1):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = Q[:, sl] @ K[:, sl].T * 0.125
            s[np.triu_indices(S, 1)] = -np.inf
            w = np.exp(s - s.max(1, keepdims=True))
            ref = (w / w.sum(1, keepdims=True)) @ V[:, sl]
            tol = 1e-5 * (1.0 + np.abs(V[:, sl]).max(0))
            assert np.all(np.abs(got[b][:, sl] - ref) <= tol), (b, hh)


@pytest.mark.parametrize("hd", [64, 128])
def test_flash_attention_live_meta_bounds_work(backend, pkg, ora, hd):
    # The grid is sized from the recorded shape (200 rows); the meta read
    # when the kernel runs says 150: rows 0..149 are attention over the first
    # 150 tokens, rows past them stay untouched, and l_cache covers 150 rows.
    # Both head sizes run the key-split kernel (a small grid).
    h = pkg.hip
    heads, S, live = 2, 200, 150
    dim = heads * hd
    q, k, v = (ora.rand_vec(S * dim, 40 + i) for i in range(3))
    out = backend.tensor(np.full(S * dim, 7.0, np.float32))
    lse = backend.tensor(np.full(S * heads, 7.0, np.float32))
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    shape = h.FlashAttnMeta(S, dim, hd, scale, 0)
    meta = _meta(backend, h.FlashAttnMeta(live, dim, hd, scale, 0))
    backend.flash_attention(backend.tensor(q), backend.tensor(k), backend.tensor(v), out, lse,
                            shape, meta)
    got = out.download().reshape(S, dim)
    ref = ora.causal_attention(q[:live * dim], k[:live * dim], v[:live * dim], live, dim, hd)
    assert np.abs(got[:live] - ref.reshape(live, dim)).max() < 1e-4
    assert np.all(got[live:] == 7.0)
    l = lse.download().reshape(S, heads)
    assert np.all(np.isfinite(l[:live])) and np.all(l[live:] == 7.0)


def test_flash_attention_c2_config(backend, pkg, ora):
    # Config 2: batch 8, 12 heads, seq 512, head_dim 64, N(0,1)
    # from seed 2, scale 1/8; sequences are row_offset slices of [8*512, 768].
    h = pkg.hip
    B, S, H, hd = 8, 512, 12, 64
    d = H * hd
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal(B * S * d, dtype=np.float32) for _ in range(3))
    tq, tk, tv = backend.tensor(q), backend.tensor(k), backend.tensor(v)
    out = backend.zeros(B * S * d)
    lse = backend.zeros(S * H)
    for b in range(B):
        shape = h.FlashAttnMeta(S, d, hd, 0.125, b * S)
        backend.flash_attention(tq, tk, tv, out, lse, shape, _meta(backend, shape))
    got = out.download().reshape(B, S * d)
    for b in (0, 5, 7):
        sl = slice(b * S * d, (b + 1) * S * d)
        ref = ora.causal_attention(q[sl], k[sl], v[sl], S, d, hd)
        assert np.abs(got[b] - ref).max() < 1e-3
    # The same 8 nodes as one batched launch, and each node's l_cache block
    # in turn.  A single node's grid is too small for the part, so it runs
    # the key-split kernel (32-query tiles, keys dealt to 4 waves, partial
    # states merged); the batched grid runs the 128-query kernel: the two
    # agree to fp32 rounding.
    out2, lse2 = backend.zeros(B * S * d), backend.zeros(B * S * H)
    shape = h.FlashAttnMeta(S, d, hd, 0.125, 0)
    backend.flash_attention_batched(tq, tk, tv, out2, lse2, shape, _meta(backend, shape), B)
    np.testing.assert_allclose(out2.download().reshape(B, S * d), got, rtol=0, atol=2e-6)
    last = h.FlashAttnMeta(S, d, hd, 0.125, (B - 1) * S)
    backend.flash_attention(tq, tk, tv, out, lse, last, _meta(backend, last))
    np.testing.assert_allclose(lse2.download()[(B - 1) * S * H:], lse.download(), rtol=0,
                               atol=2e-6)


@pytest.mark.parametrize("attn_len,heads,hd", [(1, 2, 4), (5, 3, 16), (33, 12, 64)])
def test_cached_attention_three_dispatch(backend, pkg, ora, attn_len, heads, hd):
    # cached_attention_matches_cpu_reference (emit.rs:1332-1420): grid sized
    # for max_ctx 64, meta bounds the live work; tol 1e-4.
    h = pkg.hip
    dim, max_ctx = heads * hd, 64
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    q = ora.rand_vec(dim, 1)
    kc, vc = ora.rand_vec(max_ctx * dim, 2), ora.rand_vec(max_ctx * dim, 3)
    scores = backend.zeros(heads * max_ctx)
    out = backend.zeros(dim)
    am = _meta(backend, h.AttnCachedMeta(attn_len, dim, hd))
    sm_shape = h.SoftmaxRectMeta(heads, attn_len, scale)
    tk, tv = backend.tensor(kc), backend.tensor(vc)
    backend.attn_qk_cached(backend.tensor(q), tk, scores, heads, max_ctx, am)
    backend.softmax_rect(scores, sm_shape, _meta(backend, sm_shape))
    backend.attn_av_cached(scores, tv, out, dim, am)
    s = ora.attn_qk_cached(q, kc, attn_len, dim, hd)
    p = ora.softmax_rect(s, heads, attn_len, scale)
    ref = ora.attn_av_cached(p, vc, attn_len, dim, hd)
    assert np.abs(out.download() - ref).max() < 1e-4


def test_silu_past_1d_grid_limit(backend, pkg):
    # elementwise_ops_past_1d_grid_limit (emit.rs:1473-1503).
    n = 17_000_003
    boundary = 65535 * 256
    i = np.arange(n)
    data = (((i % 1000) - 500) / 250.0).astype(np.float32)
    t = backend.tensor(data)
    backend.silu(t, n)
    out = t.download()
    for idx in (0, boundary - 1, boundary, 16_900_000, n - 1):
        v = np.float64(data[idx])
        assert abs(out[idx] - v / (1 + np.exp(-v))) < 1e-5


def test_argmax_rows(backend, pkg, ora):
    rows = np.array([[1, 4, 2, 8, 3], [1, 8, 2, 8, 3], [-np.inf] * 5], np.float32)
    out = backend.zeros(3, np.uint32)
    backend.argmax_rows(backend.tensor(rows), 3, 5, out)
    assert list(out.download(np.uint32)) == [3, 1, 0]
    big = np.random.default_rng(1).standard_normal((4, 50257)).astype(np.float32)
    big[2, 777] = big[2, 50000] = 99.0
    o2 = backend.zeros(4, np.uint32)
    backend.argmax_rows(backend.tensor(big), 4, 50257, o2)
    assert list(o2.download(np.uint32)) == [ora.argmax(r) for r in big]
    # NaN logits (sampling.rs:83-91 scans from index 0 with `>`): a NaN at
    # index 0 never loses, so the answer is 0; a NaN elsewhere never wins.
    nan = np.array([[np.nan, 4, 2, 8, 3], [1, np.nan, 9, 8, 3], [np.nan] * 5,
                    [-np.inf, np.nan, -np.inf, 2, 2]], np.float32)
    o3 = backend.zeros(4, np.uint32)
    backend.argmax_rows(backend.tensor(nan), 4, 5, o3)
    assert list(o3.download(np.uint32)) == [ora.argmax(r) for r in nan] == [0, 2, 0, 3]


def test_shader_decode_graph_replays_with_live_metas(backend, pkg, ora):
    # build_decode_layer + decode_step through the per-shader ABI, captured
    # once into a hipGraph and replayed every step after the dynamic metas
    # are rewritten (inference.rs:178-262).
    from akasha_core_amd.shader_graph import ShaderDecoder
    cfg = pkg.ModelConfig.new(97, 64, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=42)
    dec = ShaderDecoder(pkg.hip, backend, cfg, w, 16)
    ref = ora.OracleSession(cfg, w, 16)
    toks = [3, 41, 7, 96, 0, 25, 11, 12, 13, 50]
    for t in toks:
        got = dec.decode_step(t)
        exp = ref.decode_step(t)
        assert np.abs(got - exp).max() < 1e-3
        assert int(np.argmax(got)) == ora.argmax(exp)


def test_shader_decode_eager_matches_graph(backend, pkg):
    # The same launchers issued eagerly every step (capture=False) give the
    # graph replay's logits bit for bit.
    from akasha_core_amd.shader_graph import ShaderDecoder
    cfg = pkg.ModelConfig.new(97, 64, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=43)
    g = ShaderDecoder(pkg.hip, backend, cfg, w, 16)
    e = ShaderDecoder(pkg.hip, backend, cfg, w, 16, capture=False)
    for t in [5, 9, 60, 2, 2]:
        assert np.array_equal(g.decode_step(t), e.decode_step(t))
    g.close()
    e.close()


@pytest.mark.parametrize("plen", [5, 37])
def test_shader_generate_prefill_then_decode(backend, pkg, ora, plen):
    # generate on an empty cache (inference.rs:264-326): the prompt through
    # the per-shader prefill graph into the decoder's caches, then greedy
    # decode steps through the captured decode graph from position plen.
    # 5 rows run the small-m GEMV, 37 the MFMA GEMM with its K split.
    from akasha_core_amd.shader_graph import ShaderDecoder
    cfg = pkg.ModelConfig.new(97, 128, 2, 2, 48)
    w = pkg.synthetic_weights(cfg, seed=9)
    toks = [int(t) for t in ora.rand_tokens(plen, 97, 5)]
    dec = ShaderDecoder(pkg.hip, backend, cfg, w, 48)
    ref = ora.OracleSession(cfg, w, 48)
    got, exp = dec.prefill(toks), ref.prefill(toks)
    assert np.abs(got - exp).max() < 1e-3
    for _ in range(6):
        t = ora.argmax(exp)
        assert int(np.argmax(got)) == t
        got, exp = dec.decode_step(t), ref.decode_step(t)
        assert np.abs(got - exp).max() < 1e-3
    dec.close()


def test_shader_prefill_graph(backend, pkg, ora):
    from akasha_core_amd.shader_graph import shader_prefill
    cfg = pkg.ModelConfig.new(97, 128, 2, 2, 48)  # head_dim 64 -> MFMA flash
    w = pkg.synthetic_weights(cfg, seed=8)
    toks = ora.rand_tokens(37, 97, 4)
    logits, kc = shader_prefill(pkg.hip, backend, cfg, w, toks, 48)
    ref = ora.OracleSession(cfg, w, 48)
    exp = ref.prefill(toks)
    assert np.abs(logits - exp).max() < 1e-3
    np.testing.assert_allclose(kc[1], ref.k_cache(1), atol=1e-4)
