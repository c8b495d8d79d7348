"""Primitive tpu_sparse_dense_matmul_grad_with_laprop: backward pass + LaProp.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_grad_with_laprop.py:75-135``
abstract eval, ``multiple_results=True``; lowering ``:143-405``). Per touched
row, with ``decay_rate`` from ``LaPropOptimizerSpec.get_decay_rate``
(``lib/nn/embedding_spec.py:788-800``), the update body
(``sparse_dense_matmul_grad_with_laprop.py:282-340``):

  nu = nu * decay_rate + (1 - decay_rate) * (g * g + eps)
  mu = b1 * mu + (1 - b1 ** 2) ** 0.5 * (g / sqrt(nu))
  table = table - lr * mu

then the optional clipping. ``bind`` returns ``(table, mu, nu)``; see
``_optimizer`` for in-place updates and the extra keyword arguments.
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _optimizer
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          embedding_table, mu, nu, activations_grad, learning_rate, b1,
          decay_rate, eps, *_, max_ids_per_partition: int,
          max_unique_ids_per_partition: int,
          computation_name: str = "laprop_optimizer_update",
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          min_value=None, max_value=None, **kwargs):
  utils.ensure_dtype(learning_rate, np.float32, "learning_rate")
  utils.ensure_dtype(b1, np.float32, "b1")
  utils.ensure_dtype(decay_rate, np.float32, "decay_rate")
  utils.ensure_dtype(eps, np.float32, "eps")
  utils.ensure_dtype(mu, np.float32, "mu")
  utils.ensure_dtype(nu, np.float32, "nu")
  if tuple(embedding_table.shape) != tuple(mu.shape):
    raise ValueError(
        "embedding_table and mu must have equal shapes, got"
        f" {tuple(embedding_table.shape)} and {tuple(mu.shape)}")
  if tuple(embedding_table.shape) != tuple(nu.shape):
    raise ValueError(
        "embedding_table and nu must have equal shapes, got"
        f" {tuple(embedding_table.shape)} and {tuple(nu.shape)}")
  return _optimizer.apply(
      _native.OPTIMIZER_LAPROP, lhs_row_pointers, lhs_local_embedding_ids,
      lhs_local_sample_ids, lhs_gains,
      num_minibatches_per_physical_sparse_core, embedding_table, (mu, nu),
      activations_grad, (learning_rate, b1, decay_rate, eps),
      max_ids_per_partition=max_ids_per_partition,
      max_unique_ids_per_partition=max_unique_ids_per_partition,
      computation_name=computation_name, sharding_strategy=sharding_strategy,
      enable_minibatching=enable_minibatching, min_value=min_value,
      max_value=max_value, **kwargs)


tpu_sparse_dense_matmul_grad_with_laprop_primitive = utils.Primitive(
    "sparse_dense_matmul_grad_with_laprop_primitive", _impl)
tpu_sparse_dense_matmul_grad_with_laprop_primitive.multiple_results = True
