"""ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of akasha-core's inference path (akasha_oracle.c).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker / CPU baseline, never as a compute path
of the product.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_PATH = Path(__file__).resolve().parent / "liboracle.so"
_lib = None

F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")


class OraConfig(C.Structure):
    _fields_ = [("vocab_size", C.c_uint32), ("dim", C.c_uint32),
                ("num_heads", C.c_uint32), ("num_layers", C.c_uint32),
                ("ffn_hidden", C.c_uint32), ("norm_eps", C.c_float),
                ("eos_token", C.c_uint32)]


FP = C.POINTER(C.c_float)
FPP = C.POINTER(FP)


class OraWeights(C.Structure):
    _fields_ = [("embedding", FP), ("norm_1", FPP), ("qkv_proj", FPP),
                ("out_proj", FPP), ("norm_2", FPP), ("ffn_up", FPP),
                ("ffn_down", FPP), ("final_norm", FP), ("lm_head", FP)]


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not _PATH.exists():
        raise RuntimeError(f"{_PATH} missing: run `make -C oracle`")
    lib = C.CDLL(str(_PATH))
    u32, f32, sz = C.c_uint32, C.c_float, C.c_size_t
    sigs = {
        "ora_rand_vec": (None, [F32P, sz, C.c_uint64]),
        "ora_rand_tokens": (None, [U32P, sz, u32, C.c_uint64]),
        "ora_embedding": (None, [U32P, F32P, F32P, u32, u32, u32]),
        "ora_rmsnorm": (None, [F32P, F32P, F32P, u32, u32, f32]),
        "ora_matmul": (None, [F32P, F32P, F32P, u32, u32, u32]),
        "ora_matmul_add": (None, [F32P, F32P, F32P, u32, u32, u32]),
        "ora_head_gather": (None, [F32P, F32P, u32, u32, u32, u32]),
        "ora_rope": (None, [F32P, u32, u32, u32]),
        "ora_rope_offset": (None, [F32P, u32, u32, u32, u32]),
        "ora_cache_write": (None, [F32P, F32P, u32, u32, u32]),
        "ora_attn_qk_cached": (None, [F32P, F32P, F32P, u32, u32, u32]),
        "ora_softmax_rect": (None, [F32P, u32, u32, f32]),
        "ora_attn_av_cached": (None, [F32P, F32P, F32P, u32, u32, u32]),
        "ora_silu": (None, [F32P, sz]),
        "ora_causal_attention": (None, [F32P, F32P, F32P, F32P, u32, u32, u32]),
        "ora_argmax": (u32, [F32P, u32]),
        "ora_sample_token": (u32, [F32P, u32, f32, u32, f32, U32P, u32, f32, C.c_double]),
        "ora_session_new": (C.c_void_p, [C.POINTER(OraConfig), C.POINTER(OraWeights), u32]),
        "ora_session_free": (None, [C.c_void_p]),
        "ora_session_reset": (None, [C.c_void_p]),
        "ora_session_cur_len": (u32, [C.c_void_p]),
        "ora_session_prefill": (C.c_int, [C.c_void_p, U32P, u32, F32P]),
        "ora_session_decode_step": (C.c_int, [C.c_void_p, u32, F32P]),
        "ora_session_k_cache": (FP, [C.c_void_p, u32]),
        "ora_session_v_cache": (FP, [C.c_void_p, u32]),
        "ora_set_threads": (None, [C.c_int]),
        "ora_session_set_len": (None, [C.c_void_p, u32]),
        "ora_qkv_split": (None, [F32P, F32P, F32P, F32P, u32, u32, u32]),
        "ora_rope_qk": (None, [F32P, F32P, u32, u32, u32, u32]),
        "ora_add": (None, [F32P, F32P, F32P, sz]),
        "ora_residual_add": (None, [F32P, F32P, sz]),
        "ora_silu_out": (None, [F32P, F32P, sz]),
        "ora_cross_entropy": (None, [F32P, U32P, F32P, u32, u32]),
        "ora_forward_train": (f32, [C.POINTER(OraConfig), C.POINTER(OraWeights), U32P, U32P,
                                    u32, u32, F32P, C.c_void_p, C.c_void_p]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def rand_vec(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    load().ora_rand_vec(out, n, seed)
    return out


def rand_tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    load().ora_rand_tokens(out, n, vocab, seed)
    return out


def embedding(tokens, table, vocab, dim, seq_len):
    out = np.empty(seq_len * dim, np.float32)
    load().ora_embedding(np.ascontiguousarray(tokens, np.uint32), _f(table), out, vocab, dim,
                         seq_len)
    return out


def rmsnorm(x, w, rows, size, eps):
    out = np.empty(rows * size, np.float32)
    load().ora_rmsnorm(_f(x), _f(w), out, rows, size, eps)
    return out


def matmul(a, b, m, n, k):
    out = np.empty(m * n, np.float32)
    load().ora_matmul(_f(a), _f(b), out, m, n, k)
    return out


def matmul_add(a, b, c, m, n, k):
    out = _f(c).copy()
    load().ora_matmul_add(_f(a), _f(b), out, m, n, k)
    return out


def head_gather(src, seq_len, full_dim, head_dim, head_offset):
    out = np.empty(seq_len * head_dim, np.float32)
    load().ora_head_gather(_f(src), out, seq_len, full_dim, head_dim, head_offset)
    return out


def rope(x, seq_len, dim, head_dim):
    out = _f(x).copy()
    load().ora_rope(out, seq_len, dim, head_dim)
    return out


def rope_offset(x, seq_len, dim, head_dim, pos):
    out = _f(x).copy()
    load().ora_rope_offset(out, seq_len, dim, head_dim, pos)
    return out


def cache_write(src, dst, row_count, width, off):
    out = _f(dst).copy()
    load().ora_cache_write(_f(src), out, row_count, width, off)
    return out


def attn_qk_cached(q, k_cache, attn_len, dim, head_dim):
    out = np.zeros((dim // head_dim) * attn_len, np.float32)
    load().ora_attn_qk_cached(_f(q), _f(k_cache), out, attn_len, dim, head_dim)
    return out


def softmax_rect(x, num_rows, width, scale):
    out = _f(x).copy()
    load().ora_softmax_rect(out, num_rows, width, scale)
    return out


def attn_av_cached(scores, v_cache, attn_len, dim, head_dim):
    out = np.zeros(dim, np.float32)
    load().ora_attn_av_cached(_f(scores), _f(v_cache), out, attn_len, dim, head_dim)
    return out


def silu(x):
    out = _f(x).copy()
    load().ora_silu(out, out.size)
    return out


def causal_attention(q, k, v, seq_len, dim, head_dim):
    out = np.empty(seq_len * dim, np.float32)
    load().ora_causal_attention(_f(q), _f(k), _f(v), out, seq_len, dim, head_dim)
    return out


def argmax(x) -> int:
    x = _f(x)
    return int(load().ora_argmax(x, x.size))


def sample_token(logits, temperature, top_k, top_p, seen, repetition_penalty, r) -> int:
    """sampling.rs:18-81 with the draw ``r`` given (ties: lower index first)."""
    x = _f(logits)
    seen = np.ascontiguousarray(seen, np.uint32).reshape(-1)
    if seen.size == 0:
        seen = np.zeros(1, np.uint32)
        n_seen = 0
    else:
        n_seen = seen.size
    return int(load().ora_sample_token(x, x.size, float(temperature), int(top_k), float(top_p),
                                       seen, n_seen, float(repetition_penalty), float(r)))


def qkv_split(src, seq_len, full_dim, head_dim):
    n = seq_len * head_dim
    q, k, v = (np.empty(n, np.float32) for _ in range(3))
    load().ora_qkv_split(_f(src), q, k, v, seq_len, full_dim, head_dim)
    return q, k, v


def rope_qk(q, k, seq_len, dim, head_dim, row_offset):
    q, k = _f(q).copy(), _f(k).copy()
    load().ora_rope_qk(q, k, seq_len, dim, head_dim, row_offset)
    return q, k


def add(a, b):
    a, b = _f(a), _f(b)
    out = np.empty(a.size, np.float32)
    load().ora_add(a, b, out, a.size)
    return out


def residual_add(target, source):
    out, source = _f(target).copy(), _f(source)
    load().ora_residual_add(out, source, out.size)
    return out


def silu_out(x):
    x = _f(x)
    out = np.empty(x.size, np.float32)
    load().ora_silu_out(x, out, x.size)
    return out


def cross_entropy(logits, targets, vocab_size, num_rows):
    """(probs, losses): CROSS_ENTROPY's in-place probabilities and the losses."""
    x = _f(logits).copy()
    losses = np.empty(num_rows, np.float32)
    load().ora_cross_entropy(x, np.ascontiguousarray(targets, np.uint32), losses, vocab_size,
                             num_rows)
    return x, losses


def forward_train(cfg, weights, tokens, targets, batch, seq_len, want_probs=False,
                  want_hidden=False):
    """Trainer::forward + CrossEntropy: (mean_loss, losses, probs, hidden)."""
    lib = load()
    ws = [_f(w).reshape(-1) for w in weights]
    L = cfg.num_layers

    def fp(a):
        return a.ctypes.data_as(FP)

    per = [[ws[1 + 6 * l + j] for l in range(L)] for j in range(6)]
    arrs = [(FP * L)(*[fp(a) for a in per[j]]) for j in range(6)]
    w = OraWeights(fp(ws[0]), *arrs, fp(ws[1 + 6 * L]), fp(ws[2 + 6 * L]))
    c = OraConfig(cfg.vocab_size, cfg.dim, cfg.num_heads, cfg.num_layers, cfg.ffn_hidden,
                  cfg.norm_eps, cfg.eos_token)
    rows = batch * seq_len
    losses = np.empty(rows, np.float32)
    probs = np.empty((rows, cfg.vocab_size), np.float32) if want_probs else None
    hidden = np.empty((rows, cfg.dim), np.float32) if want_hidden else None
    mean = lib.ora_forward_train(C.byref(c), C.byref(w),
                                 np.ascontiguousarray(tokens, np.uint32).reshape(-1),
                                 np.ascontiguousarray(targets, np.uint32).reshape(-1),
                                 batch, seq_len, losses,
                                 probs.ctypes.data if probs is not None else None,
                                 hidden.ctypes.data if hidden is not None else None)
    return float(mean), losses, probs, hidden


def set_threads(n: int):
    load().ora_set_threads(n)


class OracleSession:
    """InferenceSession restated on the CPU (one sequence)."""

    def __init__(self, cfg, weights, max_context_len: int):
        lib = load()
        self.cfg = cfg
        self._w = [_f(w).reshape(-1) for w in weights]  # keep alive
        L = cfg.num_layers

        def fp(a):
            return a.ctypes.data_as(FP)

        per = [[self._w[1 + 6 * l + j] for l in range(L)] for j in range(6)]
        self._arrs = [(FP * L)(*[fp(a) for a in per[j]]) for j in range(6)]
        w = OraWeights(fp(self._w[0]), *self._arrs, fp(self._w[1 + 6 * L]),
                       fp(self._w[2 + 6 * L]))
        self._cfg = OraConfig(cfg.vocab_size, cfg.dim, cfg.num_heads, cfg.num_layers,
                              cfg.ffn_hidden, cfg.norm_eps, cfg.eos_token)
        self._wc = w
        self.max_context_len = max_context_len
        self.h = lib.ora_session_new(C.byref(self._cfg), C.byref(self._wc), max_context_len)

    def prefill(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.cfg.vocab_size, np.float32)
        rc = _lib.ora_session_prefill(self.h, t, t.size, out)
        if rc:
            raise RuntimeError(f"oracle prefill error {rc}")
        return out

    def decode_step(self, token: int) -> np.ndarray:
        out = np.empty(self.cfg.vocab_size, np.float32)
        rc = _lib.ora_session_decode_step(self.h, int(token), out)
        if rc:
            raise RuntimeError(f"oracle decode error {rc}")
        return out

    def cur_len(self) -> int:
        return int(_lib.ora_session_cur_len(self.h))

    def reset(self):
        _lib.ora_session_reset(self.h)

    def set_len(self, n: int):
        """Benchmark hook: treat n tokens as cached (see akasha_oracle.h)."""
        _lib.ora_session_set_len(self.h, n)

    def k_cache(self, layer: int) -> np.ndarray:
        p = _lib.ora_session_k_cache(self.h, layer)
        return np.ctypeslib.as_array(p, (self.max_context_len, self.cfg.dim)).copy()

    def v_cache(self, layer: int) -> np.ndarray:
        p = _lib.ora_session_v_cache(self.h, layer)
        return np.ctypeslib.as_array(p, (self.max_context_len, self.cfg.dim)).copy()

    def close(self):
        if self.h:
            _lib.ora_session_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
