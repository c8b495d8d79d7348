"""Shared body of the optimizer primitives with slot variables.

Every optimizer primitive of the reference lowers to the same custom call,
``SparseDenseMatmulGradOpWithOptimizerUpdate``, with the CSR, the activation
gradients, the table, its slot variables and the hyperparameters as operands
and a row-wise update function (e.g.
``lib/core/primitives/sparse_dense_matmul_grad_with_adam.py:144-405``). Here
each primitive checks its own operands as the reference's abstract eval does,
then calls ``apply``, which runs ``scemb_sparse_dense_matmul_grad_with_optimizer``
on the current stream and returns ``(table, *slots)``.

Tables and slot variables are updated in place when they are float32 CUDA
tensors (the returned tensors are those same tensors, the equivalent of
donated buffers); other inputs are copied to the GPU first and the copies are
returned.

Extra keyword arguments, as for the SGD and Adagrad primitives:
``num_sc_per_device`` / ``global_device_count``, ``csr_sorted_by_row`` (the
CSR is in the reference format's order, so one segment is read in place;
None, the default, assumes it, False sorts a copy) and
``csr_num_entries`` (entry count; picks a kernel variant, changes no
result). ``activations_grad`` may be a ``_device.RowBlocks`` (the per-feature
gradients, read in place).
"""

from __future__ import annotations

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def check_same_shape(table, named_slots, message):
  """ValueError(message(shapes)) unless every slot has the table's shape."""
  shapes = [tuple(table.shape)] + [tuple(s.shape) for _, s in named_slots]
  if any(s != shapes[0] for s in shapes[1:]):
    raise ValueError(message(*shapes))


def apply(kind: int, lhs_row_pointers, lhs_local_embedding_ids,
          lhs_local_sample_ids, lhs_gains,
          num_minibatches_per_physical_sparse_core, embedding_table, slots,
          activations_grad, hyperparameters, *, max_ids_per_partition: int,
          max_unique_ids_per_partition: int, computation_name: str,
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          min_value=None, max_value=None, num_sc_per_device=None,
          global_device_count=None, csr_sorted_by_row=None,
          csr_num_entries=None, flags: int = 0, program=None):
  """Checks shared by all primitives (utils.py:79-155), then the update."""
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
  dev_slots = [_device.device_table(x) for x in slots]
  blocks = None
  if isinstance(activations_grad, _device.RowBlocks):
    blocks, grad = activations_grad.blocks, None
    batch = activations_grad.shape[0]
  else:
    grad = _native.as_device_tensor(activations_grad, t.float32,
                                    table.device)
    batch = int(grad.shape[0])
  status = _native.status_word()
  _native.sparse_dense_matmul_grad_with_optimizer(
      csr, grad, table, kind, dev_slots, hyperparameters, batch, min_value,
      max_value, flags=flags, grad_blocks=blocks, device_status=status,
      program=program)
  _native.check_status_word(status, computation_name)
  del keep
  return (table, *dev_slots)
