"""Model shapes outside the batched decode kernels, against the CPU oracle.

The reference decodes any shape ModelConfig::new accepts (src/config.rs:15-30;
its CPU decode kernels take any head size, src/shaders/cpu.rs:144-178) and its
FLASH_ATTENTION any head_dim up to 128 (src/nn/ops/emit.rs:564-572).  The
batched decode kernels need a head size that is a multiple of 4, a dim that
is a multiple of 32 (at most 4096) and an ffn_hidden that is a multiple of 32;
other shapes decode on the generic kernels (decode_generic.hip).  Each case:
ragged prefill and greedy decode steps of a batch, sequences checked against
the oracle (identical tokens, logits within 1e-3), also with the bfloat16 KV
cache (within 2e-2) and through generate's sampler.
"""

import dataclasses

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _model(pkg, backend, dim, heads, layers, ffn, seed):
    cfg = dataclasses.replace(pkg.ModelConfig.new(173, dim, heads, layers, 40), ffn_hidden=ffn)
    w = pkg.synthetic_weights(cfg, seed=seed)
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    return cfg, w, model


# (dim, heads, ffn): head sizes 50, 6 and 34 (not multiples of 4; dim 102
# is not even a multiple of 4), dim 48 and 100 (not multiples of 32), an
# ffn_hidden of 200 (not a multiple of 32), head size 2.
SHAPES = [(100, 2, 400), (24, 4, 96), (102, 3, 408), (48, 4, 192), (100, 1, 200), (8, 4, 32)]


@pytest.mark.parametrize("dim,heads,ffn", SHAPES)
@pytest.mark.parametrize("batch", [3, 33])
def test_generic_shape_session_matches_oracle(backend, pkg, ora, dim, heads, ffn, batch):
    layers, ctx, steps = 2, 40, 4
    case = f"dim {dim} heads {heads} (hd {dim // heads}) ffn {ffn} batch {batch}"
    print(case, flush=True)
    cfg, w, model = _model(pkg, backend, dim, heads, layers, ffn, seed=dim + heads)
    r = np.random.default_rng(dim * 7 + batch)
    lens = [int(x) for x in r.integers(1, ctx - steps - 4, size=batch)]
    prompts = [r.integers(0, cfg.vocab_size, size=n).astype(np.uint32) for n in lens]
    s = pkg.hip.Session(model, ctx, batch)
    logits, nxt = s.prefill(prompts)
    got = [(logits, nxt)] + [s.decode_step(None) for _ in range(steps)]
    assert list(s.cur_len()) == [n + steps for n in lens], case
    for b in sorted({0, batch // 2, batch - 1}):
        o = ora.OracleSession(cfg, w, ctx)
        ref = o.prefill(prompts[b])
        for i in range(steps + 1):
            if i:
                ref = o.decode_step(ora.argmax(ref))
            assert np.abs(got[i][0][b] - ref).max() < TOL, f"{case}, sequence {b} step {i}"
            assert int(got[i][1][b]) == ora.argmax(ref), f"{case}, sequence {b} step {i}"
        # The cache rows the decode steps appended equal the oracle's.
        for layer in range(layers):
            n = lens[b] + steps
            kc = s.cache(layer, b, 0)[:n]
            assert np.abs(kc - o.k_cache(layer)[:n]).max() < 1e-4, f"{case}, K cache {layer}"
        o.close()
    # Greedy decode_greedy replays (a captured graph) continue the same way.
    toks = s.decode_greedy(3)
    o = ora.OracleSession(cfg, w, ctx)
    ref = o.prefill(prompts[0])
    for i in range(steps):
        ref = o.decode_step(ora.argmax(ref))
    for i in range(3):
        ref = o.decode_step(ora.argmax(ref))
        assert int(toks[i][0]) == ora.argmax(ref), f"{case}, replayed step {i}"
    o.close()
    s.close()
    model.close()


@pytest.mark.parametrize("kv16", [False, True])
def test_generic_shape_long_context(backend, pkg, ora, kv16):
    # The generic attention holds 1024 scores per pass over the keys: a
    # 1500-token prompt and decode steps past it take two passes, the
    # running maximum and sum rescaled between them.  Against the oracle
    # (logits within 1e-3, or 2e-2 with the bfloat16 cache).
    cfg, w, model = _model(pkg, backend, 100, 2, 2, 400, seed=17)
    r = np.random.default_rng(18)
    prompt = r.integers(0, cfg.vocab_size, size=(2, 1500)).astype(np.uint32)
    s = pkg.hip.Session(model, 1600, 2)
    if kv16:
        s.set_kv_bf16(True)
    logits, nxt = s.prefill(prompt)
    got = [(logits, nxt)] + [s.decode_step(None) for _ in range(3)]
    tol = 2e-2 if kv16 else TOL
    for b in range(2):
        o = ora.OracleSession(cfg, w, 1600)
        ref = o.prefill(prompt[b])
        for i in range(4):
            if i:
                ref = o.decode_step(int(got[i - 1][1][b]))
            assert np.abs(got[i][0][b] - ref).max() < tol, f"sequence {b} step {i}"
            if not kv16:
                assert int(got[i][1][b]) == ora.argmax(ref), f"sequence {b} step {i}"
        o.close()
    s.close()
    model.close()


@pytest.mark.parametrize("dim,heads,ffn", [(100, 2, 400), (102, 3, 408)])
def test_generic_shape_bf16_kv_cache(backend, pkg, ora, dim, heads, ffn):
    # The bfloat16 KV cache on the generic kernels: logits within 2e-2 of
    # the oracle's fp32 decode.
    layers, ctx, steps, batch = 2, 40, 3, 4
    cfg, w, model = _model(pkg, backend, dim, heads, layers, ffn, seed=dim)
    r = np.random.default_rng(dim)
    prompt = r.integers(0, cfg.vocab_size, size=(batch, 20)).astype(np.uint32)
    s = pkg.hip.Session(model, ctx, batch)
    s.set_kv_bf16(True)
    logits, _ = s.prefill(prompt)
    got = [logits]
    o = ora.OracleSession(cfg, w, ctx)
    ref = [o.prefill(prompt[0])]
    for _ in range(steps):
        t = ora.argmax(ref[-1])
        got.append(s.decode_step(np.full(batch, t, np.uint32))[0])
        ref.append(o.decode_step(t))
    for i in range(steps + 1):
        assert np.abs(got[i][0] - ref[i]).max() < 2e-2, f"step {i}"
    o.close()
    s.close()
    model.close()


def test_generic_shape_generate_and_errors(backend, pkg, ora):
    # generate (greedy, eos / length stops) on the generic kernels equals the
    # oracle's greedy loop; the timing entry points of the batched kernels
    # refuse such a session.
    cfg, w, model = _model(pkg, backend, 100, 2, 2, 400, seed=5)
    r = np.random.default_rng(6)
    prompt = r.integers(0, cfg.vocab_size, size=(2, 9)).astype(np.uint32)
    s = pkg.hip.Session(model, 40, 2)
    outs = s.generate(prompt, 6)
    for b in range(2):
        o = ora.OracleSession(cfg, w, 40)
        ref = o.prefill(prompt[b])
        want = []
        for _ in range(6):
            t = ora.argmax(ref)
            want.append(t)
            if t == cfg.eos_token:
                break
            ref = o.decode_step(t)
        o.close()
        assert list(outs[b]) == want, b
    with pytest.raises(pkg.hip.InvalidArgument):
        s.time_decode_kernel(1, 4)
    with pytest.raises(pkg.hip.InvalidArgument):
        s.set_fused_norm(True)
    s.close()
    model.close()
