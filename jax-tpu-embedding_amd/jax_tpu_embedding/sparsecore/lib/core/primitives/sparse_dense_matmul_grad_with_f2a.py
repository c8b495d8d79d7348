"""Primitive tpu_sparse_dense_matmul_grad_with_f2a: backward pass + F2A
(frequency-aware Adagrad).

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_grad_with_f2a.py:71-141`` abstract
eval, ``multiple_results=True``; lowering ``:149-358``). Per touched row, the
update body ``:244-290``:

  local_step = local_step + 1
  fa = min((max(global_step, 1) / local_step) ** rho, max_lr_multiplier)
  a = a + g * g
  table = table - lr * ((g * fa) / sqrt(a) + (l1 * sign(table) + l2 * table))

then the optional clipping. ``bind`` returns ``(table, accumulator,
local_step)``; see ``_optimizer`` for in-place updates and the extra keyword
arguments.
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _optimizer
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          embedding_table, accumulator, local_step, activations_grad,
          learning_rate, rho, l1_regularization_strength,
          l2_regularization_strength, max_lr_multiplier, global_step, *,
          max_ids_per_partition: int, max_unique_ids_per_partition: int,
          computation_name: str = "f2a_optimizer_update",
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          min_value=None, max_value=None, **kwargs):
  utils.ensure_dtype(embedding_table, np.float32, "embedding_table")
  utils.ensure_dtype(accumulator, np.float32, "accumulator")
  utils.ensure_dtype(local_step, np.float32, "local_step")
  utils.ensure_dtype(learning_rate, np.float32, "learning_rate")
  utils.ensure_dtype(rho, np.float32, "rho")
  utils.ensure_dtype(l1_regularization_strength, np.float32,
                     "l1_regularization_strength")
  utils.ensure_dtype(l2_regularization_strength, np.float32,
                     "l2_regularization_strength")
  utils.ensure_dtype(max_lr_multiplier, np.float32, "max_lr_multiplier")
  utils.ensure_dtype(global_step, np.float32, "global_step")
  if tuple(accumulator.shape) != tuple(embedding_table.shape):
    raise ValueError(
        f"accumulator shape {tuple(accumulator.shape)} must match "
        f"embedding_table shape {tuple(embedding_table.shape)}")
  if tuple(local_step.shape) != tuple(embedding_table.shape):
    raise ValueError(
        f"local_step shape {tuple(local_step.shape)} must match "
        f"embedding_table shape {tuple(embedding_table.shape)}")
  return _optimizer.apply(
      _native.OPTIMIZER_F2A, lhs_row_pointers, lhs_local_embedding_ids,
      lhs_local_sample_ids, lhs_gains,
      num_minibatches_per_physical_sparse_core, embedding_table,
      (accumulator, local_step), activations_grad,
      (learning_rate, rho, l1_regularization_strength,
       l2_regularization_strength, max_lr_multiplier, global_step),
      max_ids_per_partition=max_ids_per_partition,
      max_unique_ids_per_partition=max_unique_ids_per_partition,
      computation_name=computation_name, sharding_strategy=sharding_strategy,
      enable_minibatching=enable_minibatching, min_value=min_value,
      max_value=max_value, **kwargs)


tpu_sparse_dense_matmul_grad_with_f2a_primitive = utils.Primitive(
    "sparse_dense_matmul_grad_with_f2a_primitive", _impl)
tpu_sparse_dense_matmul_grad_with_f2a_primitive.multiple_results = True
