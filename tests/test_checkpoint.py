"""V3 checkpoint files (src/nn/checkpoint.rs): writer, the library's parser,
and loading into device weights.

The byte layout is pinned by a literal byte string for a tiny body, written
out by hand from checkpoint.rs:52-96 (magic, then bincode 1.x fixint fields
in declaration order, Vecs as u64 length + elements).  Loading is checked
against the uploaded arrays and by decoding with the CPU oracle; the error
cases follow checkpoint.rs:98-187.
"""


import numpy as np
import pytest


class _Cfg:
    def __init__(self, vocab_size, dim, num_heads, num_layers, seq_len, ffn_hidden):
        self.vocab_size, self.dim, self.num_heads = vocab_size, dim, num_heads
        self.num_layers, self.seq_len, self.ffn_hidden = num_layers, seq_len, ffn_hidden


# V3 body of vocab 5, dim 4, heads 2, layers 1, seq_len 8, ffn 16,
# train_step 7, schedule_step 3, params [[1.0], [2.0, -1.0]], no moments.
_TINY_V3 = bytes.fromhex(
    "414b5633"                  # "AKV3"
    "05000000" "04000000" "02000000"  # vocab_size, dim, num_heads (u32)
    "0100000000000000"          # num_layers (u64)
    "08000000" "10000000"       # seq_len, ffn_hidden (u32)
    "0700000000000000"          # train_step (u64)
    "03000000"                  # schedule_step (u32)
    "0200000000000000"          # params: Vec len 2
    "0100000000000000" "0000803f"            # [1.0]
    "0200000000000000" "00000040" "000080bf"  # [2.0, -1.0]
    "0000000000000000"          # moments: Vec len 0
)


def test_writer_byte_layout(pkg, tmp_path):
    path = tmp_path / "tiny.ckpt"
    pkg.checkpoint.save_v3(path, _Cfg(5, 4, 2, 1, 8, 16),
                           [np.array([1.0]), np.array([2.0, -1.0])],
                           train_step=7, schedule_step=3)
    assert path.read_bytes() == _TINY_V3


def test_reader_round_trip_with_moments(pkg, tmp_path):
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=5)
    mom = [(p * 0.5, p * p) for p in w]
    path = tmp_path / "m.ckpt"
    pkg.checkpoint.save_v3(path, cfg, w, moments=mom, train_step=123, schedule_step=9)
    r = pkg.checkpoint.read_v3(path)
    assert (r["vocab_size"], r["dim"], r["num_heads"], r["num_layers"], r["ffn_hidden"]) == \
        (cfg.vocab_size, cfg.dim, cfg.num_heads, cfg.num_layers, cfg.ffn_hidden)
    assert r["train_step"] == 123 and r["schedule_step"] == 9
    assert len(r["params"]) == len(w) and len(r["moments"]) == len(w)
    for a, b in zip(r["params"], w):
        np.testing.assert_array_equal(a, np.asarray(b, np.float32).reshape(-1))


def test_library_parses_header_without_a_device(pkg, tmp_path):
    path = tmp_path / "tiny.ckpt"
    path.write_bytes(_TINY_V3)
    info = pkg.hip.checkpoint_info(path)
    assert (info["vocab_size"], info["dim"], info["num_heads"], info["num_layers"],
            info["seq_len"], info["ffn_hidden"]) == (5, 4, 2, 1, 8, 16)
    assert (info["train_step"], info["schedule_step"]) == (7, 3)
    assert (info["num_params"], info["total_param_floats"], info["num_moment_pairs"]) == (2, 3, 0)


def test_library_reports_bad_files(pkg, tmp_path):
    hip = pkg.hip
    bad = tmp_path / "bad.ckpt"
    bad.write_bytes(b"AKV2" + _TINY_V3[4:])
    with pytest.raises(hip.InvalidArgument, match="is not a v3 checkpoint"):
        hip.checkpoint_info(bad)
    for cut in (3, 20, len(_TINY_V3) - 9, len(_TINY_V3) - 1):
        t = tmp_path / f"cut{cut}.ckpt"
        t.write_bytes(_TINY_V3[:cut])
        with pytest.raises(hip.FileError, match="truncated|end of file"):
            hip.checkpoint_info(t)
    with pytest.raises(hip.FileError, match="cannot open"):
        hip.checkpoint_info(tmp_path / "missing.ckpt")


# ---- device loads --------------------------------------------------------

def _model(pkg, backend, cfg):
    return pkg.hip.Model(backend, cfg)


@pytest.mark.gpu
def test_load_checkpoint_matches_arrays_and_decodes_like_oracle(backend, pkg, ora, tmp_path):
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=11)
    path = tmp_path / "w.ckpt"
    pkg.checkpoint.save_v3(path, cfg, w, train_step=42)
    m = _model(pkg, backend, cfg)
    step, has_opt = m.load_checkpoint(path)
    assert step == 42 and not has_opt
    for i, a in enumerate(w):
        np.testing.assert_array_equal(m.download_param(i), np.asarray(a, np.float32).reshape(-1))
    # Decoding with the loaded weights reproduces the oracle's greedy run.
    s = pkg.hip.Session(m, 16, 1)
    prompt = np.array([[3, 41, 7, 96, 0, 25]], np.uint32)
    logits, nxt = s.prefill(prompt)
    o = ora.OracleSession(cfg, w, 16)
    ref = o.prefill(prompt[0])
    assert np.abs(logits[0] - ref).max() < 1e-3 and int(nxt[0]) == ora.argmax(ref)
    for _ in range(4):
        logits, nxt = s.decode_step(None)
        ref = o.decode_step(ora.argmax(ref))
        assert np.abs(logits[0] - ref).max() < 1e-3 and int(nxt[0]) == ora.argmax(ref)
    o.close()


@pytest.mark.gpu
def test_load_checkpoint_errors_follow_the_reference(backend, pkg, tmp_path):
    hip = pkg.hip
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    w = pkg.synthetic_weights(cfg, seed=12)
    m = _model(pkg, backend, cfg)
    # Architecture mismatch (checkpoint.rs:111-129): nothing loaded.
    other = pkg.ModelConfig.new(97, 64, 4, 2, 16)
    p1 = tmp_path / "arch.ckpt"
    pkg.checkpoint.save_v3(p1, other, pkg.synthetic_weights(other, seed=1))
    with pytest.raises(hip.InvalidArgument, match="architecture mismatch"):
        m.load_checkpoint(p1)
    # Tensor count (checkpoint.rs:162-168).
    p2 = tmp_path / "count.ckpt"
    pkg.checkpoint.save_v3(p2, cfg, w[:-1])
    with pytest.raises(hip.InvalidArgument, match="parameter tensors, model expects"):
        m.load_checkpoint(p2)
    # Tensor size (checkpoint.rs:173-181): tensors before the bad one are loaded.
    bad = list(w)
    bad[3] = np.zeros(5, np.float32)
    p3 = tmp_path / "size.ckpt"
    pkg.checkpoint.save_v3(p3, cfg, bad)
    with pytest.raises(hip.InvalidArgument, match="checkpoint tensor 3 has 5 elements"):
        m.load_checkpoint(p3)
    np.testing.assert_array_equal(m.download_param(0), np.asarray(w[0], np.float32).reshape(-1))
    # Moment pairs (checkpoint.rs:137-145), checked after the weights.
    p4 = tmp_path / "mom.ckpt"
    pkg.checkpoint.save_v3(p4, cfg, w, moments=[(w[0], w[0])])
    with pytest.raises(hip.InvalidArgument, match="1 moment pairs, model expects"):
        m.load_checkpoint(p4)
    p5 = tmp_path / "ok.ckpt"
    pkg.checkpoint.save_v3(p5, cfg, w, moments=[(a, a) for a in w], train_step=5)
    assert m.load_checkpoint(p5) == (5, True)
    # Truncated body: an I/O error before anything is loaded.
    p6 = tmp_path / "trunc.ckpt"
    p6.write_bytes(p5.read_bytes()[:-11])
    with pytest.raises(hip.FileError):
        m.load_checkpoint(p6)
