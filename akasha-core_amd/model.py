"""ModelConfig profiles and deterministic synthetic weights.

``ModelConfig`` mirrors src/config.rs:1-61 of akasha-core (ffn_hidden = 4*dim,
norm_eps = 1e-5, eos = vocab - 1; named profiles assert head_dim == 64).

The benchmark configurations ask for weights ~N(0, 0.02) from a seed.  The
reference draws its own random init from rand's StdRng (ChaCha12), which
cannot be reproduced without Rust, so weights here come from numpy's PCG64
(``np.random.default_rng(seed)``), drawn tensor by tensor in
ModelWeights::params() order (src/nn/weights.rs:158-171).  Matrices are
N(0, std); RMSNorm gains are 1 + N(0, std) as the reference initialises them
(weights.rs:85, 94, 109).  Token ids are uniform in [0, vocab).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int
    dim: int
    num_heads: int
    num_layers: int
    seq_len: int
    ffn_hidden: int
    norm_eps: float
    eos_token: int

    @staticmethod
    def new(vocab_size: int, dim: int, num_heads: int, num_layers: int,
            seq_len: int) -> "ModelConfig":
        """ModelConfig::new (src/config.rs:15-30)."""
        assert num_layers >= 1, "At least one layer is required!"
        assert dim % num_heads == 0, "dim must be divisible by num_heads"
        return ModelConfig(vocab_size, dim, num_heads, num_layers, seq_len,
                           dim * 4, 1e-5, vocab_size - 1)

    @property
    def head_dim(self) -> int:
        return self.dim // self.num_heads

    @staticmethod
    def akasha_hall_1() -> "ModelConfig":
        """162M profile (src/config.rs:54-56)."""
        c = ModelConfig.new(50257, 768, 12, 12, 512)
        assert c.head_dim == 64
        return c

    @staticmethod
    def pidgeon() -> "ModelConfig":
        c = ModelConfig.new(50257, 320, 5, 8, 512)
        assert c.head_dim == 64
        return c

    @staticmethod
    def scaled() -> "ModelConfig":
        """The scaled benchmark architecture (dim 2048, 24 layers, 16 x 128)."""
        return ModelConfig.new(50257, 2048, 16, 24, 2048)

    def param_shapes(self):
        """Shapes in ModelWeights::params() order."""
        d, v, f = self.dim, self.vocab_size, self.ffn_hidden
        shapes = [(v, d)]
        for _ in range(self.num_layers):
            shapes += [(d,), (d, 3 * d), (d, d), (d,), (d, f), (f, d)]
        shapes += [(d,), (d, v)]
        return shapes

    def num_parameters(self) -> int:
        return int(sum(np.prod(s) for s in self.param_shapes()))


def round_to_bf16(a: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (ties to even), kept in
    float32: exactly representable in bf16."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def synthetic_weights(cfg: ModelConfig, seed: int, std: float = 0.02, bf16: bool = False):
    """Weights in params() order: matrices N(0, std), gains 1 + N(0, std).
    With ``bf16`` every value is rounded to the nearest bfloat16 (the scaled
    configuration's "bf16 weights"), still stored as float32."""
    rng = np.random.default_rng(seed)
    out = []
    for shape in cfg.param_shapes():
        a = rng.standard_normal(int(np.prod(shape)), dtype=np.float32)
        a *= np.float32(std)
        if len(shape) == 1:
            a += np.float32(1.0)
        if bf16:
            a = round_to_bf16(a)
        out.append(a.reshape(shape))
    return out


def synthetic_tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    """n uniform token ids in [0, vocab)."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, size=n, dtype=np.uint32)
