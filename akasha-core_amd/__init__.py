"""akasha-core_amd: MI355X (gfx950) backend for akasha-core's inference path.

The compute lives in libakasha_hip.so (hand-written HIP kernels + C++
runtime behind the C ABI in include/akasha_hip.h).  This package holds the
ctypes bindings (``hip``), the model profiles and synthetic-input generators
(``model``), V3 checkpoint files (``checkpoint``), the reference's per-shader
inference graphs driven through the launchers (``shader_graph``) and the
build recipe (``build``).
"""

from . import checkpoint, hip, model, shader_graph  # noqa: F401
from .model import ModelConfig, synthetic_tokens, synthetic_weights  # noqa: F401
