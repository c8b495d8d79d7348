"""Primitive tpu_sparse_dense_matmul_activation_unstack: one stacked table's
activations split into the activations of its features.

Same operand and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_activation_unstack.py:29-56``
abstract eval, ``:59-96`` lowering to the
``SparseActivationsUnstackInterleaved`` custom call). ``bind`` runs
``scemb_activation_unstack`` (a gfx950 HIP copy) on the current stream and
returns one float32 ``(per_feature_batch_sizes[i], per_feature_dims[i])``
tensor per feature, in the order given (the embedding API gives the
stack's features in row-offset order, ``embedding.py:985-1013``).

Layout ("interleaved"): the stacked activations hold one segment of
``rows / S`` rows per SparseCore, and each segment holds every feature's
slice of ``batch_f / S`` rows, features one after another. Feature f's
output row ``s * batch_f / S + i`` is stacked row
``s * rows / S + cum_f / S + i``, ``cum_f`` the batch sizes of the features
before it, columns ``[0, dim_f)``. With S = 1 this is the sequential
slicing of the reference test's mock implementation
(``primitives/tests/sparse_dense_matmul_activation_unstack_test.py:64-84``).

Extra keyword (no reference counterpart; the TPU call reads it from the
hardware): ``num_sc_per_device``, the SparseCore count S (default: the
device's).
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _check(stacked_shape, per_feature_batch_sizes, per_feature_dims,
           num_sc: int):
  if len(per_feature_batch_sizes) != len(per_feature_dims):
    raise ValueError(
        "per_feature_batch_sizes and per_feature_dims must have equal "
        f"lengths, got {len(per_feature_batch_sizes)} and "
        f"{len(per_feature_dims)}")
  if len(stacked_shape) != 2:
    raise ValueError("stacked_activations must have dim in (2,), got "
                     f"{tuple(stacked_shape)!r}")
  rows, dim = (int(d) for d in stacked_shape)
  if rows % num_sc:
    raise ValueError(
        f"stacked activations of {rows} rows do not split into {num_sc} "
        "SparseCore segments")
  total = 0
  for b, d in zip(per_feature_batch_sizes, per_feature_dims):
    if b < 0 or b % num_sc:
      raise ValueError(
          f"per-feature batch size {b} is not a non-negative multiple of "
          f"{num_sc} feature slices per device")
    if not 0 <= d <= dim:
      raise ValueError(
          f"per-feature dim {d} is outside the stacked dim {dim}")
    total += int(b)
  if total > rows:
    raise ValueError(
        f"per-feature batch sizes sum to {total}, more than the "
        f"{rows} stacked rows")


def _abstract_eval(stacked_activations, *, per_feature_batch_sizes,
                   per_feature_dims, num_sc_per_device=None):
  del stacked_activations, num_sc_per_device
  return tuple(
      utils.ShapedArray((b, d), "float32")
      for b, d in zip(per_feature_batch_sizes, per_feature_dims))


def _impl(stacked_activations, *, per_feature_batch_sizes,
          per_feature_dims, num_sc_per_device=None):
  t = _native.require_gpu()
  utils.ensure_dtype(stacked_activations, np.float32,
                     "stacked_activations")
  s, _ = _device.resolve_sparsecores(num_sc_per_device, 1)
  _check(tuple(stacked_activations.shape), per_feature_batch_sizes,
         per_feature_dims, s)
  dev = _native.device()
  stacked = _native.as_device_tensor(stacked_activations, t.float32, dev)
  rows = int(stacked.shape[0])
  seg = rows // s
  outs, blocks, cum = [], [], 0
  for b, d in zip(per_feature_batch_sizes, per_feature_dims):
    out = t.empty((int(b), int(d)), dtype=t.float32, device=dev)
    outs.append(out)
    per = int(b) // s
    for sc in range(s):
      if per and d:
        blocks.append((sc * seg + cum // s, out[sc * per:(sc + 1) * per],
                       int(d)))
    cum += int(b)
  if blocks:
    _native.activation_unstack(stacked, blocks)
  return tuple(outs)


tpu_sparse_dense_matmul_activation_unstack_primitive = utils.Primitive(
    "sparse_dense_matmul_activation_unstack", _impl,
    abstract_eval=_abstract_eval, multiple_results=True)
