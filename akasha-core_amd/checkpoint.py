"""V3 checkpoint files of akasha-core (src/nn/checkpoint.rs), host side.

``save_v3`` writes the layout ``checkpoint::save`` streams
(checkpoint.rs:52-96): the magic ``AKV3`` then one bincode 1.x ``V3Body``
in little-endian fixint encoding -- u32/u64 fields back to back, every Vec
as a u64 length followed by its elements, f32 tensors in ``params()``
order, then the AdamW (m, v) pairs.  It lets weights produced here (or
converted from elsewhere) be loaded by the reference, and by
``hip.Model.load_checkpoint``, which reads them into device memory.
``read_v3`` parses a file into numpy arrays.
"""

from __future__ import annotations

import struct

import numpy as np

MAGIC = b"AKV3"
_HEAD = struct.Struct("<IIIQIIQI")  # vocab, dim, heads, layers(u64), seq_len, ffn, train_step(u64), schedule


def _tensor(f, a) -> None:
    a = np.ascontiguousarray(a, dtype="<f4").reshape(-1)
    f.write(struct.pack("<Q", a.size))
    f.write(a.tobytes())


def save_v3(path, cfg, params, moments=None, train_step: int = 0,
            schedule_step: int = 0) -> None:
    """checkpoint::save: ``params`` in ModelWeights::params() order;
    ``moments`` is a list of (m, v) pairs in the same order, or None for a
    weights-only file."""
    moments = moments or []
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(_HEAD.pack(cfg.vocab_size, cfg.dim, cfg.num_heads, cfg.num_layers,
                           cfg.seq_len, cfg.ffn_hidden, train_step, schedule_step))
        f.write(struct.pack("<Q", len(params)))
        for p in params:
            _tensor(f, p)
        f.write(struct.pack("<Q", len(moments)))
        for m, v in moments:
            _tensor(f, m)
            _tensor(f, v)


def read_v3(path) -> dict:
    """Parse a V3 file: header fields, ``params`` and ``moments`` as float32
    arrays."""
    data = open(path, "rb").read()
    if data[:4] != MAGIC:
        raise ValueError(f"{path} is not a v3 checkpoint")
    off = 4
    vals = _HEAD.unpack_from(data, off)
    off += _HEAD.size
    out = dict(zip(("vocab_size", "dim", "num_heads", "num_layers", "seq_len",
                    "ffn_hidden", "train_step", "schedule_step"), vals))

    def tensor():
        nonlocal off
        (n,) = struct.unpack_from("<Q", data, off)
        off += 8
        a = np.frombuffer(data, dtype="<f4", count=n, offset=off).astype(np.float32)
        off += 4 * n
        return a

    (n,) = struct.unpack_from("<Q", data, off)
    off += 8
    out["params"] = [tensor() for _ in range(n)]
    (n,) = struct.unpack_from("<Q", data, off)
    off += 8
    out["moments"] = [(tensor(), tensor()) for _ in range(n)]
    return out
