"""Primitive tpu_sparse_dense_matmul_grad_with_sgd: backward pass + SGD.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_grad_with_sgd.py:51-69`` abstract
eval; lowering ``:98-232`` to ``SparseDenseMatmulGradOpWithOptimizerUpdate``
with the per-row update ``table - grad * lr``, ``:145-192``, and optional
clipping, ``primitives/utils.py:24-59``). ``bind`` runs
``scemb_sparse_dense_matmul_grad_with_sgd`` on the current stream.

The table is updated in place when it is already a float32 CUDA tensor (the
returned tensor is that same tensor, the equivalent of donating the buffer);
other inputs are copied to the GPU first and the copy is returned.

Extra keyword arguments besides ``num_sc_per_device`` /
``global_device_count``: ``csr_sorted_by_row`` declares the CSR in the
order the reference's format has (entries ascending by partition and
embedding id in each segment), with which one SparseCore segment is read in
place instead of a sorted copy; by default (None) the operands are taken to
be in that order, as every CSR the preprocessing writes is (a violated order
is reported through the status word); False makes the call sort a copy.
``csr_num_entries``, the CSR's entry count when known, picks the kernel
variant (one-hot or multi-hot batches) and changes no result.
``activations_grad`` may be a ``_device.RowBlocks``: the per-feature
gradients are then read in place (the gradient stacking of
``embedding.py:1200-1294`` fused into the kernel).
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          embedding_table, activations_grad, learning_rate, *_,
          max_ids_per_partition: int, max_unique_ids_per_partition: int,
          computation_name: str = "sgd_optimizer_update",
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          min_value=None, max_value=None, num_sc_per_device=None,
          global_device_count=None, csr_sorted_by_row=None,
          csr_num_entries=None):
  utils.ensure_dtype(learning_rate, np.float32, "learning_rate")
  utils.validate_abstract_eval_params(
      lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
      lhs_gains, num_minibatches_per_physical_sparse_core, embedding_table,
      activations_grad, max_ids_per_partition, max_unique_ids_per_partition,
      computation_name, sharding_strategy, min_value, max_value)
  nmb = sparse_dense_matmul_csr.resolve_minibatches(
      num_minibatches_per_physical_sparse_core, enable_minibatching)
  t = _native.require_gpu()
  s, ns = _device.resolve_sparsecores(num_sc_per_device, global_device_count)
  keep, csr = _device.csr_operands(lhs_row_pointers, lhs_local_embedding_ids,
                                   lhs_local_sample_ids, lhs_gains, s, ns,
                                   sorted_by_row=csr_sorted_by_row,
                                   num_entries=csr_num_entries,
                                   num_minibatches=nmb)
  table = _device.device_table(embedding_table)
  blocks = None
  if isinstance(activations_grad, _device.RowBlocks):
    blocks, grad = activations_grad.blocks, None
    batch = activations_grad.shape[0]
  else:
    grad = _native.as_device_tensor(activations_grad, t.float32,
                                    table.device)
    batch = int(grad.shape[0])
  status = _native.status_word()
  _native.sparse_dense_matmul_grad(csr, grad, table, None, learning_rate,
                                   batch, min_value, max_value,
                                   grad_blocks=blocks, device_status=status)
  _native.check_status_word(status, computation_name)
  del keep
  return table


tpu_sparse_dense_matmul_grad_with_sgd_primitive = utils.Primitive(
    "sparse_dense_matmul_grad_with_sgd", _impl)
