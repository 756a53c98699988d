"""akasha-core_amd: MI355X (gfx950) backend for akasha-core's inference path.

The compute lives in libakasha_hip.so (hand-written HIP kernels + C++
runtime behind the C ABI in include/akasha_hip.h).  This package holds the
ctypes bindings (``hip``), the model profiles and synthetic-input generators
(``model``), V3 checkpoint files (``checkpoint``) and the build recipe
(``build``).
"""

from . import checkpoint, hip, model  # noqa: F401
from .model import ModelConfig, synthetic_tokens, synthetic_weights  # noqa: F401
