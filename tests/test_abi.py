"""CPU checks of the drop-in boundary: the library loads without a GPU and
exports every entry point include/akasha_hip.h declares; meta structs have
the byte layout of src/nn/ops/meta.rs; host-side config logic."""

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "akasha_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(akh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.hip.load()
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    # The Python bindings cover the whole header too.
    assert set(names) == set(pkg.hip.EXPORTED)


def test_abi_version(pkg):
    assert pkg.hip.load().akh_abi_version() == 1


def test_meta_layouts_match_reference(pkg):
    h = pkg.hip
    # #[repr(C)] structs of u32/f32 fields (src/nn/ops/meta.rs).
    expect = {h.MatMulMeta: 12, h.NormMeta: 12, h.HeadMoveMeta: 16,
              h.AttnCachedMeta: 12, h.SoftmaxRectMeta: 12, h.RopeMeta: 16,
              h.RopeOffsetMeta: 16, h.CacheWriteMeta: 12, h.EmbeddingMeta: 12,
              h.FlashAttnMeta: 20}
    for cls, size in expect.items():
        assert C.sizeof(cls) == size, cls.__name__
    assert h.FlashAttnMeta.scale.offset == 12
    assert h.NormMeta.eps.offset == 8


def test_error_codes_follow_akasha_error(pkg):
    h = pkg.hip
    assert [h.EmptyPrompt.code, h.PromptTooLong.code, h.ContextFull.code,
            h.NoCache.code, h.CacheNotEmpty.code] == [1, 2, 3, 4, 5]
    assert all(issubclass(c, h.AkashaError) for c in h._ERRORS.values())


def test_model_profiles(pkg):
    c = pkg.ModelConfig.akasha_hall_1()
    assert (c.vocab_size, c.dim, c.num_heads, c.num_layers, c.seq_len) == (50257, 768, 12, 12, 512)
    assert c.ffn_hidden == 3072 and c.norm_eps == 1e-5 and c.eos_token == 50256
    assert c.num_parameters() == 162_148_608
    with pytest.raises(AssertionError):
        pkg.ModelConfig.new(97, 30, 4, 2, 16)


def test_synthetic_weights_are_deterministic(pkg):
    cfg = pkg.ModelConfig.new(97, 32, 4, 2, 16)
    a = pkg.synthetic_weights(cfg, 5)
    b = pkg.synthetic_weights(cfg, 5)
    assert all((x == y).all() for x, y in zip(a, b))
    assert [x.shape for x in a] == cfg.param_shapes()
    assert abs(float(a[1].mean()) - 1.0) < 0.02  # RMSNorm gain 1 + N(0, .02)
    assert abs(float(a[2].std()) - 0.02) < 0.002


def test_missing_library_fails_loudly(pkg, tmp_path):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.hip.load(tmp_path / "libakasha_hip.so")
