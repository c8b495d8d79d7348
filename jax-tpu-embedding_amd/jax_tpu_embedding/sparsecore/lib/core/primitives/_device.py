"""Operand marshalling from primitive ``bind`` arguments to the C ABI."""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.utils import utils


def resolve_sparsecores(num_sc_per_device, global_device_count):
  """SparseCores (CSR segments) per device and partitions in total."""
  if num_sc_per_device is None:
    num_sc_per_device = utils.num_sparsecores_per_device()
  g = 1 if global_device_count is None else int(global_device_count)
  return int(num_sc_per_device), int(num_sc_per_device) * g


def csr_operands(row_pointers, embedding_ids, sample_ids, gains,
                 num_sc_per_device, num_partitions, sorted_by_row=None,
                 num_entries=None, one_entry_per_row=False,
                 num_minibatches=0):
  """Device tensors for the CSR buffers plus the C struct that points at
  them (the tensors must stay alive while the struct is used).
  `sorted_by_row` declares the entries ascending by (partition, embedding
  id) inside each segment, as the preprocessing writes them; None (the
  default) takes that order from the format: the reference's CSR always has
  it (input_preprocessing_util.cc:167-208 fills each partition from the
  sorted keys), and a violation is reported through the status word. Pass
  False for buffers in another order (the backward then sorts a copy);
  `num_entries`
  the count of valid entries when known (it only picks kernel variants);
  `one_entry_per_row` at most one entry per activation row (one-hot input
  rows), which turns the grouping by activation row into a placement;
  `num_minibatches` > 0 the minibatching layout with that many minibatches
  per SparseCore (with `num_entries`, the positions past the bound on what
  the preprocessing wrote are skipped)."""
  t = _native.require_gpu()
  dev = _native.device()
  rp = _native.as_device_tensor(row_pointers, t.int32, dev).reshape(-1)
  eid = _native.as_device_tensor(embedding_ids, t.int32, dev).reshape(-1)
  sid = _native.as_device_tensor(sample_ids, t.int32, dev).reshape(-1)
  g = _native.as_device_tensor(gains, t.float32, dev).reshape(-1)
  used = 0
  if num_minibatches and num_entries:
    # Entries plus at most 7 alignment positions per (SC, minibatch,
    # partition), the last rounded up to 8.
    used = -(-(int(num_entries) + 7 * num_sc_per_device * num_minibatches *
                num_partitions) // 8) * 8
    used = used if used < 2**31 - 1 else 0
  if sorted_by_row is None:
    sorted_by_row = True
  csr = _native.make_csr(rp, eid, sid, g, num_sc_per_device, num_partitions,
                         sorted_by_row=sorted_by_row, num_entries=num_entries,
                         one_entry_per_row=one_entry_per_row,
                         num_minibatches=num_minibatches,
                         positions_used=used)
  return (rp, eid, sid, g), csr


class RowBlocks:
  """A [rows, dim] float32 activation (or activation-gradient) matrix held as
  per-feature row blocks instead of one stacked tensor: `blocks` lists
  (first_row, tensor, width) with each tensor a CUDA float32 matrix whose
  rows are stacked rows first_row.. and whose first `width` columns are the
  feature's (the rest of dim is stacking padding). The primitives accept it
  in place of the stacked matrix and read or write the blocks directly."""

  dtype = np.float32

  def __init__(self, rows: int, dim: int, blocks):
    self.shape = (int(rows), int(dim))
    self.blocks = list(blocks)

  @property
  def ndim(self) -> int:
    return 2


def device_table(table):
  """The table as a contiguous float32 CUDA tensor; a CUDA float32 input is
  returned as is so updates happen in place."""
  t = _native.require_gpu()
  return _native.as_device_tensor(table, t.float32, _native.device())
