"""Seeded random configurations of the batched session against the CPU oracle.

Each case draws a model shape (dim, heads, layers, FFN), a batch of 1..40
sequences (one or two 32-row MFMA tiles), per-sequence prompt lengths
(ragged prefill) and the session's optional knobs (fused residual add +
RMSNorm, bfloat16 weight tiles via bf16-valued weights), then checks a
few sequences' prefill and greedy decode steps against the oracle: identical
tokens, logits within 1e-3 (the fp32 bar).  The draws are fixed by the seed,
so a failure names a reproducible case.
"""

import dataclasses

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 1e-3
DIMS = [(64, 1), (64, 2), (128, 2), (128, 4), (192, 3), (256, 2), (256, 4), (384, 3)]
# Shapes the batched decode kernels do not take (head sizes 50, 6, 34, 22;
# dims not a multiple of 32): they decode on the generic kernels.
GENERIC_DIMS = [(100, 2), (24, 4), (102, 3), (88, 4), (176, 8)]


def _case(seed):
    r = np.random.default_rng(1000 + seed)
    dims = DIMS if seed < 40 else GENERIC_DIMS
    dim, heads = dims[r.integers(len(dims))]
    layers = int(r.integers(1, 4))
    ffn = int(r.choice([dim, 2 * dim, 3 * dim]))
    batch = int(r.choice([1, 3, 8, 31, 33, 40]))
    ctx = 48
    steps = int(r.integers(2, 5))
    lens = [int(x) for x in r.integers(1, ctx - steps, size=batch)]
    fused = bool(r.integers(2)) and dim % 128 == 0
    bf16 = bool(r.integers(2))
    return dim, heads, layers, ffn, batch, ctx, steps, lens, fused, bf16


@pytest.mark.parametrize("seed", range(52))
def test_random_session_matches_oracle(backend, pkg, ora, seed):
    dim, heads, layers, ffn, batch, ctx, steps, lens, fused, bf16 = _case(seed)
    case = (f"seed {seed}: dim {dim} heads {heads} layers {layers} ffn {ffn} batch {batch} "
            f"steps {steps} fused {fused} bf16 {bf16}")
    print(case, flush=True)
    cfg = dataclasses.replace(pkg.ModelConfig.new(211, dim, heads, layers, ctx), ffn_hidden=ffn)
    w = pkg.synthetic_weights(cfg, seed=seed, bf16=bf16)
    r = np.random.default_rng(seed)
    prompts = [r.integers(0, cfg.vocab_size, size=n).astype(np.uint32) for n in lens]
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    s = pkg.hip.Session(model, ctx, batch)
    if fused:
        s.set_fused_norm(True)
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
        o.close()
    s.close()
    model.close()


@pytest.mark.parametrize("dim,heads,batch", [(96, 3, 33), (160, 5, 40), (224, 2, 40)])
def test_odd_column_tile_counts_on_two_row_tiles(backend, pkg, ora, dim, heads, batch):
    """Sessions of 33..64 rows with bfloat16 weight tiles run their K-split
    decode GEMMs (qkv, out, down) two column tiles per block; widths of an odd
    number of 32-column tiles (3, 5, 7 for out and down; 9, 15, 21 for qkv)
    end the grid on a block whose second tile does not exist.  Prefill and
    greedy decode against the oracle, sequences at both row tiles."""
    layers, ctx, steps = 2, 40, 4
    case = f"dim {dim} heads {heads} batch {batch}"
    print(case, flush=True)
    cfg = dataclasses.replace(pkg.ModelConfig.new(211, dim, heads, layers, ctx), ffn_hidden=3 * dim)
    w = pkg.synthetic_weights(cfg, seed=dim, bf16=True)
    r = np.random.default_rng(dim)
    lens = [int(x) for x in r.integers(1, ctx - steps, size=batch)]
    prompts = [r.integers(0, cfg.vocab_size, size=n).astype(np.uint32) for n in lens]
    model = pkg.hip.Model(backend, cfg)
    model.upload(w)
    assert model.set_bf16_tiles(True) == 4 * layers, case  # every layer matrix
    s = pkg.hip.Session(model, ctx, batch)
    logits, nxt = s.prefill(prompts)
    got = [(logits, nxt)] + [s.decode_step(None) for _ in range(steps)]
    for b in (0, 31, 32, batch - 1):
        o = ora.OracleSession(cfg, w, ctx)
        ref = o.prefill(prompts[b])
        for i in range(steps + 1):
            if i:
                ref = o.decode_step(ora.argmax(ref))
            assert np.abs(got[i][0][b] - ref).max() < TOL, f"{case}, sequence {b} step {i}"
            assert int(got[i][1][b]) == ora.argmax(ref), f"{case}, sequence {b} step {i}"
        o.close()
    s.close()
    model.close()
