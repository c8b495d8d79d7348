"""Primitive tpu_sparse_dense_matmul_grad_with_ftrl: backward pass + FTRL.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_grad_with_ftrl.py:77-145`` abstract
eval, ``multiple_results=True``; lowering ``:153-406`` with the static
attribute ``multiply_linear_by_learning_rate``). Per touched row, the update
body ``:260-335``:

  a' = a + g * g
  dp = a' ** -lr_power - a ** -lr_power
  l' = l + lr * g - dp * table         (multiply_linear_by_learning_rate)
       l + g - (dp / lr) * table       (otherwise)
  table = (clamp(l', -l1s, l1s) - l') / den   (-l' / den when l1 == 0)

with l1s = l1 * lr (or l1) and den = a' ** -lr_power + 2 * lr * l2 + beta (or
(a' ** -lr_power + beta) / lr + 2 * l2), then the optional clipping. ``bind``
returns ``(table, accumulator, linear)``; see ``_optimizer`` for in-place
updates and the extra keyword arguments.
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _optimizer
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          embedding_table, accumulator, linear, activations_grad,
          learning_rate, learning_rate_power, l1_regularization_strength,
          l2_regularization_strength, beta, *,
          multiply_linear_by_learning_rate: bool = False,
          max_ids_per_partition: int, max_unique_ids_per_partition: int,
          computation_name: str = "ftrl_optimizer_update",
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          min_value=None, max_value=None, **kwargs):
  utils.ensure_dtype(accumulator, np.float32, "accumulator")
  utils.ensure_dtype(linear, np.float32, "linear")
  utils.ensure_dtype(learning_rate, np.float32, "learning_rate")
  utils.ensure_dtype(learning_rate_power, np.float32, "learning_rate_power")
  utils.ensure_dtype(l1_regularization_strength, np.float32,
                     "l1_regularization_strength")
  utils.ensure_dtype(l2_regularization_strength, np.float32,
                     "l2_regularization_strength")
  utils.ensure_dtype(beta, np.float32, "beta")
  shapes = (tuple(embedding_table.shape), tuple(accumulator.shape),
            tuple(linear.shape))
  if shapes[0] != shapes[1] or shapes[0] != shapes[2]:
    raise ValueError(
        "embedding_table, accumulator and linear must have identical shapes: "
        f"got {shapes[0]}, {shapes[1]}, {shapes[2]}")
  flags = (_native.OPTIMIZER_FLAG_MULTIPLY_LINEAR_BY_LR
           if bool(np.asarray(multiply_linear_by_learning_rate)) else 0)
  return _optimizer.apply(
      _native.OPTIMIZER_FTRL, lhs_row_pointers, lhs_local_embedding_ids,
      lhs_local_sample_ids, lhs_gains,
      num_minibatches_per_physical_sparse_core, embedding_table,
      (accumulator, linear), activations_grad,
      (learning_rate, learning_rate_power, l1_regularization_strength,
       l2_regularization_strength, beta),
      max_ids_per_partition=max_ids_per_partition,
      max_unique_ids_per_partition=max_unique_ids_per_partition,
      computation_name=computation_name, sharding_strategy=sharding_strategy,
      enable_minibatching=enable_minibatching, min_value=min_value,
      max_value=max_value, flags=flags, **kwargs)


tpu_sparse_dense_matmul_grad_with_ftrl_primitive = utils.Primitive(
    "sparse_dense_matmul_grad_with_ftrl_primitive", _impl)
tpu_sparse_dense_matmul_grad_with_ftrl_primitive.multiple_results = True
