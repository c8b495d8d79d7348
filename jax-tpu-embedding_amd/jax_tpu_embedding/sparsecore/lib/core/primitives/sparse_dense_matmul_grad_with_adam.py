"""Primitive tpu_sparse_dense_matmul_grad_with_adam: backward pass + Adam.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_grad_with_adam.py:76-136`` abstract
eval, ``multiple_results=True``; lowering ``:144-405``). Per touched row, with
the bias-corrected hyperparameters of ``AdamOptimizerSpec.get_hyperparameters``
(``lib/nn/embedding_spec.py:506-539``), the update body
(``sparse_dense_matmul_grad_with_adam.py:283-338``):

  m = m + (1 - beta_1) * (g - m)
  v = v + (1 - beta_2) * (g * g - v)
  table = table - (alpha_t * m) / (sqrt(v) + epsilon_hat)

then the optional clipping. ``bind`` returns ``(table, momentum, velocity)``;
see ``_optimizer`` for in-place updates and the extra keyword arguments.
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _optimizer
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          embedding_table, momentum, velocity, activations_grad, alpha_t,
          beta_1, beta_2, epsilon_hat, *_, max_ids_per_partition: int,
          max_unique_ids_per_partition: int,
          computation_name: str = "adam_optimizer_update",
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          min_value=None, max_value=None, **kwargs):
  utils.ensure_dtype(alpha_t, np.float32, "alpha_t")
  utils.ensure_dtype(beta_1, np.float32, "beta_1")
  utils.ensure_dtype(beta_2, np.float32, "beta_2")
  utils.ensure_dtype(epsilon_hat, np.float32, "epsilon_hat")
  utils.ensure_dtype(momentum, np.float32, "momentum")
  utils.ensure_dtype(velocity, np.float32, "velocity")
  if tuple(embedding_table.shape) != tuple(velocity.shape):
    raise ValueError(
        "embedding_table and velocity must have equal shapes, got"
        f" {tuple(embedding_table.shape)} and {tuple(velocity.shape)}")
  if tuple(embedding_table.shape) != tuple(momentum.shape):
    raise ValueError(
        "embedding_table and momentum must have equal shapes, got"
        f" {tuple(embedding_table.shape)} and {tuple(momentum.shape)}")
  return _optimizer.apply(
      _native.OPTIMIZER_ADAM, lhs_row_pointers, lhs_local_embedding_ids,
      lhs_local_sample_ids, lhs_gains,
      num_minibatches_per_physical_sparse_core, embedding_table,
      (momentum, velocity), activations_grad,
      (alpha_t, beta_1, beta_2, epsilon_hat),
      max_ids_per_partition=max_ids_per_partition,
      max_unique_ids_per_partition=max_unique_ids_per_partition,
      computation_name=computation_name, sharding_strategy=sharding_strategy,
      enable_minibatching=enable_minibatching, min_value=min_value,
      max_value=max_value, **kwargs)


tpu_sparse_dense_matmul_grad_with_adam_primitive = utils.Primitive(
    "sparse_dense_matmul_grad_with_adam_primitive", _impl)
tpu_sparse_dense_matmul_grad_with_adam_primitive.multiple_results = True
