"""tkmi -- MI355X-native transformer-layer forward (gfx950 HIP kernels behind a C ABI).

Public surface mirrors the reference's drop-in module (src/optimized.py):
``OptimizedTransformer``, ``OptimizerSettings``, ``configure``,
``active_settings``; the parameter tree ``BaselineTransformer`` and
``TransformerConfig``; and the kernel wrappers in ``tkmi.ops``.
"""

from .model import OptimizedTransformer, OptimizerSettings, active_settings, configure
from .modules import BaselineTransformer, TransformerConfig
from . import ops

__all__ = [
    "OptimizedTransformer",
    "OptimizerSettings",
    "configure",
    "active_settings",
    "BaselineTransformer",
    "TransformerConfig",
    "ops",
]
