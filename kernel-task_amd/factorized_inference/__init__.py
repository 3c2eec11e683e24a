"""MI355X-native three-core tensor-ring linear operator.

Same public names as the reference's package (src/factorized_inference/__init__.py:1-18):
TRSpec, make_cores, tr_forward_reference, materialize_dense_weight, dense_forward,
prepare_optimized, tr_forward_optimized.
"""
from .reference import (
    TRSpec,
    dense_forward,
    make_cores,
    materialize_dense_weight,
    tr_forward_reference,
)
from .submission import prepare_optimized, tr_forward_optimized

__all__ = [
    "TRSpec",
    "dense_forward",
    "make_cores",
    "materialize_dense_weight",
    "tr_forward_reference",
    "tr_forward_optimized",
    "prepare_optimized",
]
