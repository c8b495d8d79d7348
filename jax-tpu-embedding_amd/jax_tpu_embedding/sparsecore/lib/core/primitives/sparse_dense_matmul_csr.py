"""Primitive tpu_sparse_dense_matmul_csr: the forward embedding lookup.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_csr.py:47-62`` abstract eval,
``:114-202`` lowering to the ``SparseDenseMatmulOp`` custom call); ``bind``
validates like the abstract eval and runs ``scemb_sparse_dense_matmul``
(gfx950 HIP) on the current stream. Result: float32 activations of shape
``(device_batch_size, dim)`` (``(device_batch_size,)`` for a 1-D table).

Extra keyword arguments (no reference counterpart; the TPU op reads them from
the hardware): ``num_sc_per_device`` and ``global_device_count`` give the CSR
segment / partition counts (defaults: the device's SparseCore count, 1);
``lookup_view`` is an optional ``_native.LookupView`` of the same CSR (built
by the preprocessing), which spares the call its grouping sort. A view built
for another batch size or table height is ignored. ``activation_blocks``
(a ``_device.RowBlocks``) makes the call write every activation row into its
feature's block (the unstacking of ``embedding.py:903-1044`` fused into the
kernel) and return that object instead of a stacked matrix. In validation
mode (``_native.set_validation``) the call checks the kernels' status word
and raises RuntimeError on out-of-range entries or a mislabelled stream.
``csr_num_entries``, the
CSR's entry count when known, picks the kernel variant (one-hot or
multi-hot batches) and changes no result.
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def resolve_minibatches(num_minibatches, enable_minibatching: bool) -> int:
  """The CSR layout the operands are in: 0 without minibatching (one block
  of row pointers per SparseCore; the count must then be 1, a device scalar
  is not read back), else the minibatch count (1 to 64) of the minibatching
  layout ("SparseDenseMatmulWithMinibatchingOp",
  sparse_dense_matmul_csr.py:171-192 of the reference)."""
  if not enable_minibatching:
    if isinstance(num_minibatches, (int, np.integer, np.ndarray)):
      if int(np.asarray(num_minibatches).reshape(())) != 1:
        raise ValueError("num_minibatches must be 1 without minibatching")
    return 0
  if hasattr(num_minibatches, "item") and not isinstance(
      num_minibatches, (np.ndarray, np.generic)):
    n = int(num_minibatches.reshape(()).item())  # device scalar: one read
  else:
    n = int(np.asarray(num_minibatches).reshape(()))
  if not 1 <= n <= _native.MAX_MINIBATCHES:
    raise ValueError(f"num_minibatches must be in [1, 64], got {n}")
  return n


def _validate_quantization(quantization_config):
  if quantization_config is None:
    return
  q_min, q_max, q_buckets = quantization_config
  if q_buckets < 2:
    raise ValueError(
        f"quantization_num_buckets must be at least 2, got {q_buckets}")
  if q_min >= q_max:
    raise ValueError(
        "quantization_min_valuemust be less than quantization_max_value,"
        f" got {q_min} and {q_max}")


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          embedding_table, *, device_batch_size: int,
          max_ids_per_partition: int, max_unique_ids_per_partition: int,
          sharding_strategy: int = 1, quantization_config=None,
          enable_minibatching: bool = False, num_sc_per_device=None,
          global_device_count=None, lookup_view=None, csr_num_entries=None,
          activation_blocks=None):
  utils.validate_abstract_eval_params(
      lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
      lhs_gains, num_minibatches_per_physical_sparse_core, embedding_table,
      activations_grad=None,
      max_ids_per_partition=max_ids_per_partition,
      max_unique_ids_per_partition=max_unique_ids_per_partition,
      computation_name="fwd-pass", sharding_strategy=sharding_strategy)
  _validate_quantization(quantization_config)
  if quantization_config is not None:
    raise NotImplementedError("quantized tables are not supported yet")
  nmb = resolve_minibatches(num_minibatches_per_physical_sparse_core,
                            enable_minibatching)
  t = _native.require_gpu()
  s, ns = _device.resolve_sparsecores(num_sc_per_device, global_device_count)
  keep, csr = _device.csr_operands(lhs_row_pointers, lhs_local_embedding_ids,
                                   lhs_local_sample_ids, lhs_gains, s, ns,
                                   num_entries=csr_num_entries,
                                   num_minibatches=nmb)
  table = _device.device_table(embedding_table)
  shape = ((device_batch_size,) if table.dim() == 1 else
           (device_batch_size, int(table.shape[1])))
  if lookup_view is not None and (
      lookup_view.device_batch_size != int(device_batch_size) or
      lookup_view.table_rows != int(table.shape[0])):
    lookup_view = None
  if activation_blocks is not None:
    if tuple(activation_blocks.shape) != (int(device_batch_size),
                                          int(table.shape[-1])) or (
                                              table.dim() != 2):
      raise ValueError(
          f"activation_blocks of shape {activation_blocks.shape} do not match "
          f"the activations ({device_batch_size}, {table.shape[-1]})")
    status = _native.status_word()
    _native.sparse_dense_matmul_to_blocks(csr, table, activation_blocks.blocks,
                                          int(device_batch_size),
                                          view=lookup_view,
                                          device_status=status)
    _native.check_status_word(status, "sparse_dense_matmul")
    del keep
    return activation_blocks
  out = t.empty(shape, dtype=t.float32, device=table.device)
  status = _native.status_word()
  _native.sparse_dense_matmul(csr, table, out, int(device_batch_size),
                              view=lookup_view, device_status=status)
  _native.check_status_word(status, "sparse_dense_matmul")
  del keep
  return out


tpu_sparse_dense_matmul_csr_primitive = utils.Primitive(
    "sparse_dense_matmul_csr", _impl)
