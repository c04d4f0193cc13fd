"""granulelayer_amd: MI355X (gfx950) sparse projection -> activation -> pool layer.

Public API mirrors sparse_pooling/__init__.py (the reference package) for the Mode-A hot path:
``SparsePoolingLayer``, ``PoolingConfig``, ``LevelSpec``, ``PhysicalPlan``, ``SparseLayout``,
``init_parameters``, ``CoverTopK16Layer`` (sparse_pooling/cover_topk16.py) and ``FusedAdamW``
(sparse_pooling/optim.py).  The compute runs in the HIP
library granulelayer_amd/lib/libgranulelayer_amd.so through its C ABI
(include/granulelayer_amd.h).
"""
from .config import LevelSpec, PhysicalPlan, PoolingConfig
from .cover_topk16 import CoverTopK16Layer
from .layer import SparsePoolingLayer
from .layout import SparseLayout, init_parameters
from .optim import FusedAdamW

__all__ = ["SparsePoolingLayer", "PoolingConfig", "LevelSpec", "PhysicalPlan", "SparseLayout", "init_parameters",
           "CoverTopK16Layer", "FusedAdamW"]
