"""MantisNet leaf evaluation on MI355X: the stone/window/cell graph network
for Hexo, with its custom operators as HIP kernels for gfx950.

The public surface mirrors the reference package's hot path
(python/mantisnet/mantisnet/__init__.py): ``MantisConfig``, ``MantisNet``,
``ModelOutput``, ``Batch`` and the batch constructors.
"""

from .builder import (
    MODEL_REPR_VERSION,
    TERN_DEC_CLASSES,
    TERN_OCC_CLASSES,
    TERN_PATTERNS,
    Batch,
    batch_from_arrays,
    build_batch_prefixes,
    collate_positions,
    collate_prefixes,
    decode_batch,
    encode_position,
)
from .model import PRODUCTION, MantisConfig, MantisNet, ModelOutput, compose_acting_q, compose_q
from . import library  # noqa: E402,F401  registers the mantisnet:: operators

__all__ = [
    "MODEL_REPR_VERSION",
    "TERN_DEC_CLASSES",
    "TERN_OCC_CLASSES",
    "TERN_PATTERNS",
    "Batch",
    "batch_from_arrays",
    "build_batch_prefixes",
    "collate_positions",
    "collate_prefixes",
    "decode_batch",
    "encode_position",
    "MantisConfig",
    "MantisNet",
    "ModelOutput",
    "PRODUCTION",
    "compose_q",
    "compose_acting_q",
]
