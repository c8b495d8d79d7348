"""Primitive tpu_sparse_dense_matmul_gradient_stack: the activation
gradients of a stacked table's features stacked into one matrix.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_gradient_stack.py:29-43``
abstract eval, ``:46-86`` lowering to the ``SparseGradientsStackInterleaved``
custom call). ``bind`` runs ``scemb_gradient_stack`` (a gfx950 HIP copy) on
the current stream and returns the float32
``(stacked_batch_size, stacked_feature_dim)`` gradient.

The operands are the features' gradients in row-offset order, each
``(batch_f, dim_f)`` with ``dim_f <= stacked_feature_dim`` (the embedding
API passes them padded to the stack's dim, ``embedding.py:1200-1217``).
Layout ("interleaved", the inverse of the activation unstacking): one
segment of ``stacked_batch_size / S`` rows per SparseCore, each holding
every feature's slice of ``batch_f / S`` rows, features one after another;
columns past a feature's width, and rows past the features, are zero. With
S = 1 this is the concatenation of the reference test's mock implementation
(``primitives/tests/sparse_dense_matmul_gradient_stack_test.py:63-87``).

Extra keyword (no reference counterpart; the TPU call reads it from the
hardware): ``num_sc_per_device``, the SparseCore count S (default: the
device's).
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils


def _abstract_eval(*unstacked_gradients, stacked_batch_size: int,
                   stacked_feature_dim: int, num_sc_per_device=None):
  del unstacked_gradients, num_sc_per_device
  return utils.ShapedArray((stacked_batch_size, stacked_feature_dim),
                           "float32")


def _impl(*unstacked_gradients, stacked_batch_size: int,
          stacked_feature_dim: int, num_sc_per_device=None):
  t = _native.require_gpu()
  if not unstacked_gradients:
    raise ValueError("at least one gradient is required")
  s, _ = _device.resolve_sparsecores(num_sc_per_device, 1)
  rows, dim = int(stacked_batch_size), int(stacked_feature_dim)
  if rows < 0 or dim <= 0 or rows % s:
    raise ValueError(
        f"stacked gradient ({rows}, {dim}) does not split into {s} "
        "SparseCore segments")
  dev = _native.device()
  seg = rows // s
  blocks, cum, keep = [], 0, []
  for i, g in enumerate(unstacked_gradients):
    utils.ensure_dtype(g, np.float32, f"unstacked_gradients[{i}]")
    utils.ensure_dim(g, 2, f"unstacked_gradients[{i}]")
    g = _native.as_device_tensor(g, t.float32, dev)
    keep.append(g)
    b, d = int(g.shape[0]), int(g.shape[1])
    if b % s:
      raise ValueError(
          f"gradient {i} has {b} rows, not a multiple of {s} feature slices "
          "per device")
    if d > dim:
      raise ValueError(
          f"gradient {i} is {d} wide, more than the stacked dim {dim}")
    per = b // s
    for sc in range(s):
      if per:
        blocks.append((sc * seg + cum // s, g[sc * per:(sc + 1) * per], d))
    cum += b
  if cum > rows:
    raise ValueError(
        f"the gradients hold {cum} rows, more than the {rows} stacked rows")
  out = t.empty((rows, dim), dtype=t.float32, device=dev)
  _native.gradient_stack(blocks, out)
  del keep
  return out


tpu_sparse_dense_matmul_gradient_stack_primitive = utils.Primitive(
    "sparse_dense_matmul_gradient_stack", _impl,
    abstract_eval=_abstract_eval)
