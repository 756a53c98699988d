"""ctypes bindings of libakasha_hip.so (include/akasha_hip.h).

Host-side mirror of the reference's inference interfaces, for tests and the
benchmark.  Names, argument meaning and errors follow akasha-core:

* ``Backend`` ~ wilupgu's HipBackend (src/main.rs:366) + Tensor I/O;
* ``Backend.<shader>`` ~ the ``ops::*_with`` emitters (src/nn/ops/emit.rs)
  with metas laid out as src/nn/ops/meta.rs;
* ``Model`` ~ ModelWeights (src/nn/weights.rs), parameters in params() order;
* ``Session`` ~ InferenceSession (src/nn/inference.rs) over ``batch``
  independent sequences; failures raise ``AkashaError`` subclasses named
  after the reference's enum variants (src/lib.rs:10-17).

All compute runs in the HIP library.  There is no CPU fallback: if the
library is missing, ``load()`` raises.
"""

from __future__ import annotations

import atexit
import ctypes as C
import os
import weakref
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "libakasha_hip.so"
_lib = None

AKH_OK = 0


class AkashaError(RuntimeError):
    """Base of the reference's AkashaError variants (src/lib.rs:10-17)."""

    code = -1


class EmptyPrompt(AkashaError):
    code = 1


class PromptTooLong(AkashaError):
    code = 2


class ContextFull(AkashaError):
    code = 3


class NoCache(AkashaError):
    code = 4


class CacheNotEmpty(AkashaError):
    code = 5


class InvalidArgument(AkashaError):
    """A precondition the reference enforces with assert! (a panic)."""

    code = 6


class HipError(AkashaError):
    code = 7


class FileError(AkashaError):
    """A checkpoint file cannot be opened, read, or is truncated."""

    code = 8


_ERRORS = {c.code: c for c in (EmptyPrompt, PromptTooLong, ContextFull,
                               NoCache, CacheNotEmpty, InvalidArgument,
                               HipError, FileError)}


class Sampling(C.Structure):
    """akh_sampling: sample_token's parameters (src/nn/sampling.rs:18-25)."""

    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float)]


class CheckpointInfo(C.Structure):
    """akh_checkpoint_info_t: V3Body's header (src/nn/checkpoint.rs:20-35)."""

    _fields_ = [("vocab_size", C.c_uint32), ("dim", C.c_uint32), ("num_heads", C.c_uint32),
                ("num_layers", C.c_uint64), ("seq_len", C.c_uint32), ("ffn_hidden", C.c_uint32),
                ("train_step", C.c_uint64), ("schedule_step", C.c_uint32),
                ("num_params", C.c_uint64), ("total_param_floats", C.c_uint64),
                ("num_moment_pairs", C.c_uint64)]


# ---- meta structs (src/nn/ops/meta.rs) -----------------------------------

class MatMulMeta(C.Structure):
    _fields_ = [("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32)]


class NormMeta(C.Structure):
    _fields_ = [("seq_len", C.c_uint32), ("size", C.c_uint32), ("eps", C.c_float)]


class HeadMoveMeta(C.Structure):
    _fields_ = [("seq_len", C.c_uint32), ("full_dim", C.c_uint32),
                ("head_dim", C.c_uint32), ("head_offset", C.c_uint32)]


class AttnCachedMeta(C.Structure):
    _fields_ = [("attn_len", C.c_uint32), ("dim", C.c_uint32), ("head_dim", C.c_uint32)]


class SoftmaxRectMeta(C.Structure):
    _fields_ = [("num_rows", C.c_uint32), ("width", C.c_uint32), ("scale", C.c_float)]


class RopeMeta(C.Structure):
    _fields_ = [("seq_len", C.c_uint32), ("dim", C.c_uint32),
                ("head_dim", C.c_uint32), ("row_offset", C.c_uint32)]


class RopeOffsetMeta(C.Structure):
    _fields_ = [("seq_len", C.c_uint32), ("dim", C.c_uint32),
                ("head_dim", C.c_uint32), ("pos", C.c_uint32)]


class CacheWriteMeta(C.Structure):
    _fields_ = [("row_count", C.c_uint32), ("width", C.c_uint32),
                ("dst_row_offset", C.c_uint32)]


class EmbeddingMeta(C.Structure):
    _fields_ = [("vocab_size", C.c_uint32), ("dim", C.c_uint32), ("seq_len", C.c_uint32)]


class FlashAttnMeta(C.Structure):
    _fields_ = [("seq_len", C.c_uint32), ("dim", C.c_uint32), ("head_dim", C.c_uint32),
                ("scale", C.c_float), ("row_offset", C.c_uint32)]


class CrossEntropyMeta(C.Structure):
    _fields_ = [("vocab_size", C.c_uint32), ("num_rows", C.c_uint32)]


class ModelConfigC(C.Structure):
    _fields_ = [("vocab_size", C.c_uint32), ("dim", C.c_uint32),
                ("num_heads", C.c_uint32), ("num_layers", C.c_uint32),
                ("ffn_hidden", C.c_uint32), ("norm_eps", C.c_float),
                ("eos_token", C.c_uint32)]


P = C.c_void_p
U32 = C.c_uint32
ST = C.c_int

# name -> (restype, argtypes)
_SIGS = {
    "akh_abi_version": (C.c_int, []),
    "akh_last_error": (C.c_char_p, []),
    "akh_backend_new": (ST, [C.c_int, C.POINTER(P)]),
    "akh_backend_free": (None, [P]),
    "akh_synchronize": (ST, [P]),
    "akh_tensor_alloc": (ST, [P, C.c_size_t, C.POINTER(P)]),
    "akh_tensor_free": (ST, [P, P]),
    "akh_tensor_upload": (ST, [P, P, P, C.c_size_t]),
    "akh_tensor_from_host": (ST, [P, P, C.c_size_t, C.POINTER(P)]),
    "akh_tensor_download": (ST, [P, P, P, C.c_size_t]),
    "akh_graph_begin": (ST, [P]),
    "akh_graph_end": (ST, [P, C.POINTER(P)]),
    "akh_graph_execute": (ST, [P]),
    "akh_graph_free": (None, [P]),
    "akh_embedding": (ST, [P, P, P, P, EmbeddingMeta, P]),
    "akh_rmsnorm": (ST, [P, P, P, P, NormMeta, P]),
    "akh_matmul": (ST, [P, P, P, P, MatMulMeta, P]),
    "akh_matmul_add": (ST, [P, P, P, P, MatMulMeta, P]),
    "akh_head_gather": (ST, [P, P, P, HeadMoveMeta, P]),
    "akh_rope": (ST, [P, P, RopeMeta, P]),
    "akh_rope_offset": (ST, [P, P, RopeOffsetMeta, P]),
    "akh_cache_write": (ST, [P, P, P, CacheWriteMeta, P]),
    "akh_flash_attention": (ST, [P, P, P, P, P, P, FlashAttnMeta, P]),
    "akh_flash_attention_batched": (ST, [P, P, P, P, P, P, FlashAttnMeta, P, U32]),
    "akh_attn_qk_cached": (ST, [P, P, P, P, U32, U32, P]),
    "akh_softmax_rect": (ST, [P, P, SoftmaxRectMeta, P]),
    "akh_attn_av_cached": (ST, [P, P, P, P, U32, P]),
    "akh_silu": (ST, [P, P, U32]),
    "akh_qkv_split": (ST, [P, P, P, P, P, HeadMoveMeta, P]),
    "akh_rope_qk": (ST, [P, P, P, RopeMeta, P]),
    "akh_add": (ST, [P, P, P, P, U32]),
    "akh_residual_add": (ST, [P, P, P, U32]),
    "akh_silu_out": (ST, [P, P, P, U32]),
    "akh_cross_entropy": (ST, [P, P, P, P, CrossEntropyMeta, P]),
    "akh_forward_new": (ST, [P, U32, U32, C.POINTER(P)]),
    "akh_forward_free": (None, [P]),
    "akh_forward_loss": (ST, [P, P, P, P, C.POINTER(C.c_float)]),
    "akh_forward_probs": (ST, [P, U32, U32, P]),
    "akh_forward_hidden": (ST, [P, P]),
    "akh_argmax_rows": (ST, [P, P, U32, U32, P]),
    "akh_sample_rows": (ST, [P, P, U32, U32, Sampling, P, U32, P, P, P]),
    "akh_sample_rows_noalloc": (ST, [P, P, U32, U32, Sampling, P, U32, P, P, P]),
    "akh_model_new": (ST, [P, C.POINTER(ModelConfigC), C.POINTER(P)]),
    "akh_model_free": (None, [P]),
    "akh_model_num_params": (U32, [P]),
    "akh_model_param": (ST, [P, U32, C.POINTER(P), C.POINTER(C.c_size_t)]),
    "akh_model_upload_param": (ST, [P, U32, P, C.c_size_t]),
    "akh_model_set_bf16_tiles": (ST, [P, C.c_int, P]),
    "akh_model_set_prefill_bf16": (ST, [P, C.c_int]),
    "akh_model_set_prefill_x6": (ST, [P, C.c_int]),
    "akh_model_set_prefill_split": (ST, [P, C.c_int]),
    "akh_model_prefill_split": (C.c_int, [P]),
    "akh_checkpoint_info": (ST, [C.c_char_p, C.POINTER(CheckpointInfo)]),
    "akh_model_load_checkpoint": (ST, [P, C.c_char_p, C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_int)]),
    "akh_session_new": (ST, [P, U32, U32, C.POINTER(P)]),
    "akh_session_free": (None, [P]),
    "akh_session_reset": (ST, [P]),
    "akh_session_cur_len": (ST, [P, P]),
    "akh_session_prefill": (ST, [P, P, U32, P, P]),
    "akh_session_decode_step": (ST, [P, P, P, P]),
    "akh_session_decode_greedy": (ST, [P, U32, P]),
    "akh_session_generate": (ST, [P, P, U32, U32, Sampling, P, P, P]),
    "akh_session_generate_ragged": (ST, [P, P, P, U32, Sampling, P, P, P]),
    "akh_session_prefill_ragged": (ST, [P, P, P, P, P]),
    "akh_session_truncate": (ST, [P, U32]),
    "akh_session_set_len": (ST, [P, U32]),
    "akh_session_fill_cache_synthetic": (ST, [P, U32, C.c_uint64]),
    "akh_session_set_kv_bf16": (ST, [P, C.c_int]),
    "akh_session_take_cache": (ST, [P, U32, P, P, C.POINTER(U32), C.POINTER(C.c_int)]),
    "akh_session_replace_cache": (ST, [P, U32, P, P, U32]),
    "akh_session_download_cache": (ST, [P, U32, U32, C.c_int, P]),
    "akh_timer_start": (ST, [P]),
    "akh_timer_stop": (ST, [P, C.POINTER(C.c_float)]),
    "akh_session_time_decode_kernel": (ST, [P, C.c_int, U32, C.POINTER(C.c_float)]),
    "akh_session_time_decode_attn": (ST, [P, U32, C.POINTER(C.c_float)]),
    "akh_session_decode_launches": (ST, [P, C.POINTER(U32)]),
    "akh_session_set_fused_norm": (ST, [P, C.c_int]),
}

EXPORTED = tuple(_SIGS)


def lib_path() -> Path:
    return _LIB_PATH


def checkpoint_info(path) -> dict:
    """Header and tensor-list shape of a V3 checkpoint (no device needed)."""
    lib = load()
    info = CheckpointInfo()
    _check(lib.akh_checkpoint_info(os.fsencode(path), C.byref(info)), "checkpoint_info")
    return {name: getattr(info, name) for name, _ in CheckpointInfo._fields_}


def load(path: str | os.PathLike | None = None):
    """Load libakasha_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else _LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it with __graft_entry__.build() "
                           "(there is no CPU fallback)")
    lib = C.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.akh_abi_version() != 1:
        raise RuntimeError("libakasha_hip ABI version mismatch")
    if path is None:
        _lib = lib
    return lib


def _check(status: int, what: str = ""):
    if status != AKH_OK:
        msg = _lib.akh_last_error().decode(errors="replace")
        cls = _ERRORS.get(status, AkashaError)
        raise cls(f"{what}: {msg}" if what else msg)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class DeviceTensor:
    """A device allocation (Tensor<HipBackend>): raw pointer + byte size."""

    def __init__(self, backend: "Backend", nbytes: int, host=None):
        """Zeroed device memory, or (host: a buffer of nbytes) a copy of host
        (akh_tensor_from_host, Tensor::init_from_cpu)."""
        self.backend = backend
        self.nbytes = nbytes
        out = C.c_void_p()
        if host is None:
            _check(_lib.akh_tensor_alloc(backend.handle, nbytes, C.byref(out)), "alloc")
        else:
            _check(_lib.akh_tensor_from_host(backend.handle, host, nbytes, C.byref(out)),
                   "from_host")
        self.ptr = out
        backend._adopt(self)

    def upload(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes, "upload larger than tensor"
        _check(_lib.akh_tensor_upload(self.backend.handle, self.ptr, _ptr(arr), arr.nbytes),
               "upload")
        return self

    def download(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        n = self.nbytes // np.dtype(dtype).itemsize if count is None else count
        out = np.empty(n, dtype=dtype)
        _check(_lib.akh_tensor_download(self.backend.handle, _ptr(out), self.ptr,
                                        out.nbytes), "download")
        return out

    def offset(self, byte_offset: int) -> C.c_void_p:
        return C.c_void_p(self.ptr.value + byte_offset)

    def free(self):
        if self.ptr and self.backend.handle:
            _check(_lib.akh_tensor_free(self.backend.handle, self.ptr), "free")
        self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.backend.handle:
                _lib.akh_tensor_free(self.backend.handle, self.ptr)
                self.ptr = None
        except Exception:
            pass


def _p(x):
    if isinstance(x, DeviceTensor):
        return x.ptr
    return x


# Backends still open when the interpreter exits are closed (children
# first) before the HIP runtime's own teardown, which would otherwise run
# before the garbage collector frees them in arbitrary order.
_LIVE_BACKENDS = weakref.WeakSet()


@atexit.register
def _close_live_backends():
    for be in list(_LIVE_BACKENDS):
        try:
            be.close()
        except Exception:
            pass


class Backend:
    """HipBackend: one device, one stream (default priority)."""

    def __init__(self, device: int = 0):
        load()
        h = C.c_void_p()
        _check(_lib.akh_backend_new(device, C.byref(h)), "backend_new")
        self.handle = h
        # Sessions, models and tensors must be released before the backend.
        self._children = weakref.WeakSet()
        _LIVE_BACKENDS.add(self)

    def _adopt(self, obj):
        self._children.add(obj)
        return obj

    def close(self):
        if self.handle:
            kids = list(self._children)
            for kind in (Session, Model, Graph, DeviceTensor):
                for k in kids:
                    if isinstance(k, kind):
                        k.close() if not isinstance(k, DeviceTensor) else k.free()
            _lib.akh_backend_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # tensors
    def tensor(self, data: np.ndarray) -> DeviceTensor:
        """Tensor::init_from_cpu."""
        data = np.ascontiguousarray(data)
        if data.nbytes == 0:
            return DeviceTensor(self, 4)
        return DeviceTensor(self, data.nbytes, _ptr(data))

    def zeros(self, n: int, dtype=np.float32) -> DeviceTensor:
        return DeviceTensor(self, max(n * np.dtype(dtype).itemsize, 4))

    def meta(self, m: C.Structure) -> DeviceTensor:
        """KernelMeta::upload (src/nn/ops/meta.rs:4-11)."""
        return DeviceTensor(self, C.sizeof(m), C.cast(C.pointer(m), C.c_void_p))

    def write_meta(self, t: DeviceTensor, m: C.Structure):
        """KernelMeta::write_to (src/nn/ops/meta.rs:12-15)."""
        _check(_lib.akh_tensor_upload(self.handle, t.ptr, C.byref(m), C.sizeof(m)), "meta")

    def synchronize(self):
        _check(_lib.akh_synchronize(self.handle), "synchronize")

    # graphs
    def graph_begin(self):
        _check(_lib.akh_graph_begin(self.handle), "graph_begin")

    def graph_end(self) -> "Graph":
        g = C.c_void_p()
        _check(_lib.akh_graph_end(self.handle, C.byref(g)), "graph_end")
        return self._adopt(Graph(g))

    # timing
    def timer_start(self):
        _check(_lib.akh_timer_start(self.handle), "timer_start")

    def timer_stop(self) -> float:
        ms = C.c_float()
        _check(_lib.akh_timer_stop(self.handle, C.byref(ms)), "timer_stop")
        return ms.value

    # shaders (ops::*_with)
    def embedding(self, tokens, table, out, shape: EmbeddingMeta, meta):
        _check(_lib.akh_embedding(self.handle, _p(tokens), _p(table), _p(out), shape, _p(meta)),
               "embedding")

    def rmsnorm(self, x, w, out, shape: NormMeta, meta):
        _check(_lib.akh_rmsnorm(self.handle, _p(x), _p(w), _p(out), shape, _p(meta)), "rmsnorm")

    def matmul(self, a, b, c, shape: MatMulMeta, meta):
        _check(_lib.akh_matmul(self.handle, _p(a), _p(b), _p(c), shape, _p(meta)), "matmul")

    def matmul_add(self, a, b, c, shape: MatMulMeta, meta):
        _check(_lib.akh_matmul_add(self.handle, _p(a), _p(b), _p(c), shape, _p(meta)),
               "matmul_add")

    def head_gather(self, src, dst, shape: HeadMoveMeta, meta):
        _check(_lib.akh_head_gather(self.handle, _p(src), _p(dst), shape, _p(meta)),
               "head_gather")

    def rope(self, buf, shape: RopeMeta, meta):
        _check(_lib.akh_rope(self.handle, _p(buf), shape, _p(meta)), "rope")

    def rope_offset(self, buf, shape: RopeOffsetMeta, meta):
        _check(_lib.akh_rope_offset(self.handle, _p(buf), shape, _p(meta)), "rope_offset")

    def cache_write(self, src, cache, shape: CacheWriteMeta, meta):
        _check(_lib.akh_cache_write(self.handle, _p(src), _p(cache), shape, _p(meta)),
               "cache_write")

    def flash_attention_batched(self, q, k, v, out, l_cache, shape: FlashAttnMeta, meta, batch):
        _check(_lib.akh_flash_attention_batched(self.handle, _p(q), _p(k), _p(v), _p(out),
                                                _p(l_cache), shape, _p(meta), batch),
               "flash_attention_batched")

    def flash_attention(self, q, k, v, out, l_cache, shape: FlashAttnMeta, meta):
        _check(_lib.akh_flash_attention(self.handle, _p(q), _p(k), _p(v), _p(out),
                                        _p(l_cache), shape, _p(meta)), "flash_attention")

    def attn_qk_cached(self, q, k_cache, scores, num_heads, max_attn_len, meta):
        _check(_lib.akh_attn_qk_cached(self.handle, _p(q), _p(k_cache), _p(scores),
                                       num_heads, max_attn_len, _p(meta)), "attn_qk_cached")

    def softmax_rect(self, scores, shape: SoftmaxRectMeta, meta):
        _check(_lib.akh_softmax_rect(self.handle, _p(scores), shape, _p(meta)), "softmax_rect")

    def attn_av_cached(self, scores, v_cache, out, dim, meta):
        _check(_lib.akh_attn_av_cached(self.handle, _p(scores), _p(v_cache), _p(out), dim,
                                       _p(meta)), "attn_av_cached")

    def silu(self, buf, length):
        _check(_lib.akh_silu(self.handle, _p(buf), length), "silu")

    def qkv_split(self, src, q, k, v, shape: HeadMoveMeta, meta):
        _check(_lib.akh_qkv_split(self.handle, _p(src), _p(q), _p(k), _p(v), shape, _p(meta)),
               "qkv_split")

    def rope_qk(self, q, k, shape: RopeMeta, meta):
        _check(_lib.akh_rope_qk(self.handle, _p(q), _p(k), shape, _p(meta)), "rope_qk")

    def add(self, a, b, out, length):
        _check(_lib.akh_add(self.handle, _p(a), _p(b), _p(out), length), "add")

    def residual_add(self, target, source, length):
        _check(_lib.akh_residual_add(self.handle, _p(target), _p(source), length), "residual_add")

    def silu_out(self, x, out, length):
        _check(_lib.akh_silu_out(self.handle, _p(x), _p(out), length), "silu_out")

    def cross_entropy(self, logits, targets, losses, shape: CrossEntropyMeta, meta):
        _check(_lib.akh_cross_entropy(self.handle, _p(logits), _p(targets), _p(losses), shape,
                                      _p(meta)), "cross_entropy")

    def argmax_rows(self, logits, rows, n, out):
        _check(_lib.akh_argmax_rows(self.handle, _p(logits), rows, n, _p(out)), "argmax_rows")

    def sample_rows(self, logits, rows, n, out, temperature=0.0, top_k=0, top_p=1.0,
                    repetition_penalty=1.0, seen=None, seen_stride=0, seen_len=None,
                    uniforms=None):
        """sample_token per row of device logits (device buffers throughout)."""
        sp = Sampling(temperature, top_k, top_p, repetition_penalty)
        _check(_lib.akh_sample_rows(self.handle, _p(logits), rows, n, sp,
                                    _p(seen) if seen is not None else None, seen_stride,
                                    _p(seen_len) if seen_len is not None else None,
                                    _p(uniforms) if uniforms is not None else None, _p(out)),
               "sample_rows")

    def sample_rows_noalloc(self, logits, rows, n, out, temperature=0.0, top_k=0, top_p=1.0,
                            repetition_penalty=1.0, seen=None, seen_stride=0, seen_len=None,
                            uniforms=None):
        """sample_rows on the device's fixed workspace: allocates nothing
        (rows * n <= 2^21)."""
        sp = Sampling(temperature, top_k, top_p, repetition_penalty)
        _check(_lib.akh_sample_rows_noalloc(self.handle, _p(logits), rows, n, sp,
                                            _p(seen) if seen is not None else None, seen_stride,
                                            _p(seen_len) if seen_len is not None else None,
                                            _p(uniforms) if uniforms is not None else None,
                                            _p(out)),
               "sample_rows_noalloc")


class Graph:
    def __init__(self, handle):
        self.handle = handle

    def execute(self):
        _check(_lib.akh_graph_execute(self.handle), "graph_execute")

    def close(self):
        if self.handle:
            _lib.akh_graph_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """ModelWeights on the device (src/nn/weights.rs)."""

    def __init__(self, backend: Backend, cfg):
        self.backend = backend
        self.cfg = cfg
        c = ModelConfigC(cfg.vocab_size, cfg.dim, cfg.num_heads, cfg.num_layers,
                         cfg.ffn_hidden, cfg.norm_eps, cfg.eos_token)
        h = C.c_void_p()
        _check(_lib.akh_model_new(backend.handle, C.byref(c), C.byref(h)), "model_new")
        self.handle = h
        backend._adopt(self)

    @property
    def num_params(self) -> int:
        return _lib.akh_model_num_params(self.handle)

    def param(self, index: int):
        dev, cnt = C.c_void_p(), C.c_size_t()
        _check(_lib.akh_model_param(self.handle, index, C.byref(dev), C.byref(cnt)), "param")
        return dev, cnt.value

    def upload(self, params):
        """Upload a list of float32 arrays in params() order."""
        assert len(params) == self.num_params
        for i, a in enumerate(params):
            a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
            _check(_lib.akh_model_upload_param(self.handle, i, _ptr(a), a.size), f"param {i}")

    def set_bf16_tiles(self, allow: bool) -> int:
        """Allow or forbid bfloat16 decode tiles (re-tiles every matrix);
        returns how many matrices are tiled in bfloat16."""
        n = U32()
        _check(_lib.akh_model_set_bf16_tiles(self.handle, 1 if allow else 0, C.byref(n)),
               "set_bf16_tiles")
        return n.value

    SPLIT_NONE, SPLIT_X6, SPLIT_H3 = 0, 1, 2

    def set_prefill_split(self, kind: int):
        """Kernels of the f32 prefill GEMMs, all fp32-accurate: SPLIT_H3 (two
        fp16 terms per operand, three products; the default where dim and
        ffn_hidden are multiples of 8), SPLIT_X6 (three bfloat16 terms, six
        products) or SPLIT_NONE (the fp32 MFMAs)."""
        _check(_lib.akh_model_set_prefill_split(self.handle, int(kind)), "set_prefill_split")

    def prefill_split(self) -> int:
        return int(_lib.akh_model_prefill_split(self.handle))

    def set_prefill_x6(self, enable: bool):
        """set_prefill_split(SPLIT_X6 if enable else SPLIT_NONE)."""
        _check(_lib.akh_model_set_prefill_x6(self.handle, 1 if enable else 0),
               "set_prefill_x6")

    def set_prefill_bf16(self, enable: bool):
        """The optional bf16-MFMA prefill (logits within 2e-2 of f32)."""
        _check(_lib.akh_model_set_prefill_bf16(self.handle, 1 if enable else 0),
               "set_prefill_bf16")

    def download_param(self, index: int) -> np.ndarray:
        """Host copy of parameter ``index`` (reference layout)."""
        dev, n = self.param(index)
        out = np.empty(n, np.float32)
        _check(_lib.akh_tensor_download(self.backend.handle, _ptr(out), dev, out.nbytes),
               "download_param")
        return out

    def load_checkpoint(self, path):
        """checkpoint::load of a V3 file; returns (train_step, has_optimizer)."""
        step, opt = C.c_uint64(), C.c_int()
        _check(_lib.akh_model_load_checkpoint(self.handle, os.fsencode(path), C.byref(step),
                                              C.byref(opt)), "load_checkpoint")
        return step.value, bool(opt.value)

    def close(self):
        if self.handle:
            _lib.akh_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Forward:
    """Trainer::forward + CrossEntropy over batch x seq_len rows
    (src/nn/train.rs:256-275), on the prefill kernels."""

    def __init__(self, model: "Model", batch: int, seq_len: int):
        self.model, self.batch, self.seq_len = model, batch, seq_len
        h = P()
        _check(_lib.akh_forward_new(model.handle, batch, seq_len, C.byref(h)), "forward_new")
        self.handle = h

    def loss(self, tokens, targets):
        """(mean_loss, losses [batch * seq_len])."""
        t = np.ascontiguousarray(tokens, np.uint32).reshape(-1)
        g = np.ascontiguousarray(targets, np.uint32).reshape(-1)
        assert t.size == g.size == self.batch * self.seq_len
        losses = np.empty(t.size, np.float32)
        mean = C.c_float()
        _check(_lib.akh_forward_loss(self.handle, _ptr(t), _ptr(g), _ptr(losses),
                                     C.byref(mean)), "forward_loss")
        return mean.value, losses

    def probs(self, row0: int, n: int) -> np.ndarray:
        out = np.empty((n, self.model.cfg.vocab_size), np.float32)
        _check(_lib.akh_forward_probs(self.handle, row0, n, _ptr(out)), "forward_probs")
        return out

    def hidden(self) -> np.ndarray:
        out = np.empty((self.batch * self.seq_len, self.model.cfg.dim), np.float32)
        _check(_lib.akh_forward_hidden(self.handle, _ptr(out)), "forward_hidden")
        return out

    def close(self):
        if self.handle:
            _lib.akh_forward_free(self.handle)
            self.handle = None


class Session:
    """InferenceSession over ``batch`` independent sequences."""

    def __init__(self, model: Model, max_context_len: int, batch: int = 1):
        self.model = model
        self.batch = batch
        self.max_context_len = max_context_len
        h = C.c_void_p()
        _check(_lib.akh_session_new(model.handle, max_context_len, batch, C.byref(h)),
               "session_new")
        self.handle = h
        model.backend._adopt(self)

    def reset(self):
        _check(_lib.akh_session_reset(self.handle), "reset")

    def cur_len(self) -> np.ndarray:
        out = np.zeros(self.batch, dtype=np.uint32)
        _check(_lib.akh_session_cur_len(self.handle, _ptr(out)), "cur_len")
        return out

    @staticmethod
    def _packed(prompts, batch):
        """A list of per-sequence prompts -> (tokens back to back, lengths)."""
        if len(prompts) != batch:
            raise InvalidArgument(f"{len(prompts)} prompts for {batch} sequences")
        lens = np.array([len(p) for p in prompts], np.uint32)
        toks = (np.concatenate([np.asarray(p, np.uint32).reshape(-1) for p in prompts])
                if lens.sum() else np.zeros(1, np.uint32))
        return np.ascontiguousarray(toks, np.uint32), lens

    def prefill(self, tokens, want_logits: bool = True):
        """tokens [batch, S], or a list of batch prompts of any lengths
        (akh_session_prefill_ragged) -> (logits [batch, vocab] or None,
        next [batch])."""
        logits = (np.empty((self.batch, self.model.cfg.vocab_size), np.float32)
                  if want_logits else None)
        nxt = np.empty(self.batch, np.uint32)
        lp = _ptr(logits) if logits is not None else None
        if isinstance(tokens, (list, tuple)):
            t, lens = self._packed(tokens, self.batch)
            _check(_lib.akh_session_prefill_ragged(self.handle, _ptr(t), _ptr(lens), lp,
                                                   _ptr(nxt)), "prefill_ragged")
            return logits, nxt
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(self.batch, -1))
        _check(_lib.akh_session_prefill(self.handle, _ptr(t), t.shape[1], lp, _ptr(nxt)),
               "prefill")
        return logits, nxt

    def decode_step(self, tokens=None, want_logits: bool = True):
        """tokens [batch] (None: feed the previous greedy tokens)."""
        tp = None
        if tokens is not None:
            t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(self.batch))
            tp = _ptr(t)
        logits = (np.empty((self.batch, self.model.cfg.vocab_size), np.float32)
                  if want_logits else None)
        nxt = np.empty(self.batch, np.uint32)
        _check(_lib.akh_session_decode_step(self.handle, tp,
                                            _ptr(logits) if logits is not None else None,
                                            _ptr(nxt)), "decode_step")
        return logits, nxt

    def decode_greedy(self, steps: int, want_tokens: bool = True):
        out = np.empty((steps, self.batch), np.uint32) if want_tokens else None
        _check(_lib.akh_session_decode_greedy(self.handle, steps,
                                              _ptr(out) if out is not None else None),
               "decode_greedy")
        return out

    def generate(self, prompt, max_new_tokens: int, temperature: float = 0.0, top_k: int = 0,
                 top_p: float = 1.0, repetition_penalty: float = 1.0, uniforms=None):
        """InferenceSession::generate per sequence (token ids).  ``prompt`` is
        [batch, prompt_len], or a list of batch prompts of any lengths
        (akh_session_generate_ragged); ``uniforms`` [max_new_tokens, batch]
        holds the draws standing in for rand::random() (needed when
        temperature > 0).  Returns a list of uint32 arrays, one per
        sequence."""
        out = np.zeros((self.batch, max(1, max_new_tokens)), np.uint32)
        counts = np.zeros(self.batch, np.uint32)
        uni = None
        if uniforms is not None:
            uni = np.ascontiguousarray(uniforms, np.float64).reshape(max_new_tokens, self.batch)
        sp = Sampling(temperature, top_k, top_p, repetition_penalty)
        up = _ptr(uni) if uni is not None else None
        if isinstance(prompt, (list, tuple)):
            t, lens = self._packed(prompt, self.batch)
            _check(_lib.akh_session_generate_ragged(self.handle, _ptr(t), _ptr(lens),
                                                    max_new_tokens, sp, up, _ptr(out),
                                                    _ptr(counts)), "generate_ragged")
        else:
            prompt = np.ascontiguousarray(prompt, np.uint32).reshape(self.batch, -1)
            _check(_lib.akh_session_generate(self.handle, _ptr(prompt), prompt.shape[1],
                                             max_new_tokens, sp, up, _ptr(out), _ptr(counts)),
                   "generate")
        return [out[b, :counts[b]].copy() for b in range(self.batch)]

    def truncate(self, length: int):
        _check(_lib.akh_session_truncate(self.handle, length), "truncate")

    def set_len(self, length: int):
        """Cache::cur_len = length for every sequence (rows untouched)."""
        _check(_lib.akh_session_set_len(self.handle, length), "set_len")

    def fill_cache_synthetic(self, length: int, seed: int):
        """Rows [0, length) of every K/V cache filled with N(0, 1) values
        (hash of seed), then cur_len = length (measurement only)."""
        _check(_lib.akh_session_fill_cache_synthetic(self.handle, length, seed),
               "fill_cache_synthetic")

    def set_kv_bf16(self, enable: bool):
        """bfloat16 KV cache (the optional bf16 path); caches must be empty."""
        _check(_lib.akh_session_set_kv_bf16(self.handle, 1 if enable else 0), "set_kv_bf16")

    def take_cache(self, seq: int):
        """take_cache for one sequence: (k, v, cur_len) or None if it had none."""
        c = self.model.cfg
        shape = (c.num_layers, self.max_context_len, c.dim)
        k, v = np.empty(shape, np.float32), np.empty(shape, np.float32)
        n, had = U32(), C.c_int()
        _check(_lib.akh_session_take_cache(self.handle, seq, _ptr(k), _ptr(v), C.byref(n),
                                           C.byref(had)), "take_cache")
        return (k, v, n.value) if had.value else None

    def replace_cache(self, seq: int, k, v, cur_len: int):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        _check(_lib.akh_session_replace_cache(self.handle, seq, _ptr(k), _ptr(v), cur_len),
               "replace_cache")

    def cache(self, layer: int, seq: int, which: int) -> np.ndarray:
        out = np.empty((self.max_context_len, self.model.cfg.dim), np.float32)
        _check(_lib.akh_session_download_cache(self.handle, layer, seq, which, _ptr(out)),
               "download_cache")
        return out

    def time_decode_kernel(self, kernel: int, reps: int) -> float:
        ms = C.c_float()
        _check(_lib.akh_session_time_decode_kernel(self.handle, kernel, reps, C.byref(ms)),
               "time_decode_kernel")
        return ms.value

    def time_decode_attn(self, reps: int) -> float:
        """Mean duration (ms) of the decode attention dispatch alone, from
        events the dispatches carry (no gaps between launches)."""
        ms = C.c_float()
        _check(_lib.akh_session_time_decode_attn(self.handle, reps, C.byref(ms)),
               "time_decode_attn")
        return ms.value

    def decode_launches(self) -> int:
        """Kernel launches in one decode step (nodes of the step's graph)."""
        n = U32()
        _check(_lib.akh_session_decode_launches(self.handle, C.byref(n)), "decode_launches")
        return n.value

    def set_fused_norm(self, enable: bool):
        """Fold the residual adds + RMSNorms into the decode GEMMs (five
        launches per layer instead of seven; off by default)."""
        _check(_lib.akh_session_set_fused_norm(self.handle, int(bool(enable))), "set_fused_norm")

    def close(self):
        if self.handle:
            _lib.akh_session_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
