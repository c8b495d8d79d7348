"""Primitive tpu_sparse_dense_matmul_grad_with_adagrad_momentum.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_grad_with_adagrad_momentum.py:
76-136`` abstract eval, ``multiple_results=True``; lowering ``:144-382``). Per
touched row, the update body ``:256-311``:

  a = a + g * g                      if beta2 == 1
      beta2 * a + (1 - beta2) * g * g otherwise
  s = (a + epsilon) ** (-1 / exponent) * g
  m = momentum * m + s
  table = table - lr * (momentum * m + s if use_nesterov else m)

then the optional clipping. ``bind`` returns ``(table, accumulator,
momentum)``; see ``_optimizer`` for in-place updates and the extra keyword
arguments.
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _optimizer
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          embedding_table, accumulator, momentum, activations_grad,
          learning_rate, momentum_param, beta2, epsilon, exponent,
          use_nesterov, *_, max_ids_per_partition: int,
          max_unique_ids_per_partition: int,
          computation_name: str = "adagrad_momentum_optimizer_update",
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          min_value=None, max_value=None, **kwargs):
  utils.ensure_dtype(accumulator, np.float32, "accumulator")
  utils.ensure_dtype(momentum, np.float32, "momentum")
  utils.ensure_dtype(learning_rate, np.float32, "learning_rate")
  utils.ensure_dtype(momentum_param, np.float32, "momentum_param")
  utils.ensure_dtype(beta2, np.float32, "beta2")
  utils.ensure_dtype(epsilon, np.float32, "epsilon")
  utils.ensure_dtype(exponent, np.float32, "exponent")
  utils.ensure_dtype(use_nesterov, np.bool_, "use_nesterov")
  shapes = (tuple(embedding_table.shape), tuple(accumulator.shape),
            tuple(momentum.shape))
  if shapes[0] != shapes[1] or shapes[0] != shapes[2]:
    raise ValueError(
        "embedding_table, accumulator and momentum must have identical "
        f"shapes: got {shapes[0]}, {shapes[1]}, {shapes[2]}")
  nesterov = use_nesterov
  if not hasattr(nesterov, "data_ptr"):
    nesterov = 1.0 if bool(np.asarray(use_nesterov)) else 0.0
  return _optimizer.apply(
      _native.OPTIMIZER_ADAGRAD_MOMENTUM, lhs_row_pointers,
      lhs_local_embedding_ids, lhs_local_sample_ids, lhs_gains,
      num_minibatches_per_physical_sparse_core, embedding_table,
      (accumulator, momentum), activations_grad,
      (learning_rate, momentum_param, beta2, epsilon, exponent, nesterov),
      max_ids_per_partition=max_ids_per_partition,
      max_unique_ids_per_partition=max_unique_ids_per_partition,
      computation_name=computation_name, sharding_strategy=sharding_strategy,
      enable_minibatching=enable_minibatching, min_value=min_value,
      max_value=max_value, **kwargs)


tpu_sparse_dense_matmul_grad_with_adagrad_momentum_primitive = (
    utils.Primitive("sparse_dense_matmul_grad_with_adagrad_momentum_primitive",
                    _impl))
tpu_sparse_dense_matmul_grad_with_adagrad_momentum_primitive.multiple_results = True
