"""Operand validation shared by the primitives.

Restates the checks of ``lib/core/primitives/utils.py:62-155`` (dtypes, ranks,
matching minor dimensions, sharding strategy, positive limits, clip bounds)
with the same ``ValueError`` messages, applied to torch tensors / numpy
arrays before anything is launched.
"""

from __future__ import annotations

import numpy as np

_NP_OF = {
    "torch.int32": np.int32,
    "torch.int64": np.int64,
    "torch.float32": np.float32,
    "torch.float64": np.float64,
    "torch.float16": np.float16,
    "torch.bfloat16": None,
    "torch.uint8": np.uint8,
    "torch.bool": np.bool_,
}


def _dtype(x):
  # Python scalars are weakly typed (JAX's default 32-bit mode): int -> int32,
  # float -> float32.
  if isinstance(x, bool):
    return np.bool_
  if isinstance(x, int):
    return np.int32
  if isinstance(x, float):
    return np.float32
  if hasattr(x, "dtype"):
    d = x.dtype
    s = str(d)
    if s.startswith("torch."):
      return _NP_OF.get(s, s)
    return np.dtype(d).type
  return np.asarray(x).dtype.type


def _shape(x):
  return tuple(x.shape) if hasattr(x, "shape") else np.shape(x)


def ensure_dtype(check, expected_type, object_name: str):
  if _dtype(check) != expected_type:
    raise ValueError(
        f"{object_name} must have type {np.dtype(expected_type)!r}, got "
        f"{_dtype(check)!r}")


def ensure_dim(check, expected_dim, object_name: str):
  expected = (expected_dim,) if isinstance(expected_dim, int) else expected_dim
  if len(_shape(check)) not in expected:
    raise ValueError(
        f"{object_name} must have dim in {expected!r}, got {_shape(check)!r}")


def get_embedding_dim(val) -> int:
  s = _shape(val)
  return s[1] if len(s) > 1 else 1


def validate_abstract_eval_params(
    lhs_row_pointers,
    lhs_local_embedding_ids,
    lhs_local_sample_ids,
    lhs_gains,
    num_minibatches_per_physical_sparse_core,
    embedding_table,
    activations_grad,
    max_ids_per_partition: int,
    max_unique_ids_per_partition: int,
    computation_name: str,
    sharding_strategy: int,
    min_value: float | None = None,
    max_value: float | None = None,
):
  """Checks common to every primitive (utils.py:79-155)."""
  ensure_dtype(lhs_row_pointers, np.int32, "lhs_row_pointers")
  ensure_dtype(lhs_local_sample_ids, np.int32, "lhs_local_sample_ids")
  ensure_dtype(lhs_local_embedding_ids, np.int32, "lhs_local_embedding_ids")
  ensure_dtype(lhs_gains, np.float32, "lhs_gains")
  ensure_dtype(num_minibatches_per_physical_sparse_core, np.int32,
               "num_minibatches_per_physical_sparse_core")
  ensure_dtype(embedding_table, np.float32, "embedding_table")
  if activations_grad is not None:
    ensure_dtype(activations_grad, np.float32, "activations_grad")
  ensure_dim(lhs_row_pointers, 1, "lhs_row_pointers")
  ensure_dim(embedding_table, (1, 2), "embedding_table")
  ensure_dim(num_minibatches_per_physical_sparse_core, 0,
             "num_minibatches_per_physical_sparse_core")
  if activations_grad is not None:
    ensure_dim(activations_grad, (1, 2), "activations_grad")
  if (_shape(lhs_local_sample_ids) != _shape(lhs_local_embedding_ids) or
      _shape(lhs_gains) != _shape(lhs_local_embedding_ids) or
      len(_shape(lhs_local_sample_ids)) != 1):
    raise ValueError(
        "LHS sample IDs, embedding IDs, and gains must all have "
        "equal rank 1 shapes, got shapes "
        f"{_shape(lhs_local_sample_ids)}, {_shape(lhs_local_embedding_ids)} "
        f"and {_shape(lhs_gains)}")
  if activations_grad is not None:
    if get_embedding_dim(embedding_table) != get_embedding_dim(
        activations_grad):
      raise ValueError(
          "embedding_table and activations_grad must have equal feature "
          f"(minor) dimensions, got {_shape(embedding_table)}, "
          f"{_shape(activations_grad)}")
  if sharding_strategy != 1:
    raise ValueError(
        f"sharding_strategy must be MOD (1), got {sharding_strategy}")
  if max_ids_per_partition <= 0:
    raise ValueError(
        f"max_ids_per_partition must be positive, got {max_ids_per_partition}")
  if max_unique_ids_per_partition <= 0:
    raise ValueError("max_unique_ids_per_partition must be positive, got"
                     f" {max_unique_ids_per_partition}")
  if not computation_name:
    raise ValueError("computation_name must be non-empty")
  if min_value is not None and max_value is not None and min_value > max_value:
    raise ValueError(
        "min_value must be less than or equal to max_value, got"
        f" {min_value} and {max_value}")


class ShapedArray(tuple):
  """Shape and dtype of a result (jax.core.ShapedArray's two fields)."""

  def __new__(cls, shape, dtype):
    return super().__new__(cls, (tuple(int(d) for d in shape),
                                 np.dtype(dtype)))

  @property
  def shape(self):
    return self[0]

  @property
  def dtype(self):
    return self[1]


class Primitive:
  """Named operation with a ``bind`` entry point, like jex.core.Primitive.

  ``bind`` validates operands and runs the HIP implementation eagerly on the
  current torch stream. ``abstract_eval`` (when the primitive defines one)
  gives the results' ShapedArrays from the operands' shapes alone, without a
  device.
  """

  def __init__(self, name: str, impl, abstract_eval=None,
               multiple_results: bool = False):
    self.name = name
    self._impl = impl
    self._abstract_eval = abstract_eval
    self.multiple_results = multiple_results

  def bind(self, *args, **kwargs):
    return self._impl(*args, **kwargs)

  def abstract_eval(self, *args, **kwargs):
    if self._abstract_eval is None:
      raise NotImplementedError(f"{self.name} has no abstract evaluation")
    return self._abstract_eval(*args, **kwargs)

  def __repr__(self):
    return self.name
