"""Single-feature preprocessing entry point (lib/core/input_preprocessing.py).

The reference module is a readable Python restatement used by the primitive
tests (``primitives/tests/*``): one feature batch (dense 2-D array or a list
of samples) with per-id weights, partitioned over the mesh's SparseCores,
deduplicated per (column, sample) with the weights summed, packed into the
CSR-wrapped COO buffers (reference ``input_preprocessing.py:126-286``, entry
``:290-383``). Here the same computation runs on the GPU through the stacked
preprocessing pipeline (libscemb.so) with one feature, the sum combiner (a
gain is the summed weight) and a buffer of
``roundup8(max_ids_per_partition) * num_sc_per_device * num_scs`` entries.

Differences from the reference module, all documented behaviour of the C++
path this build follows: duplicate weights are summed in float32 in sorted
order (the Python module sums in float64 before the float32 cast), and ids
must be non-negative. Limits are checked as in the reference
(``_validate_partition_map``, ``:96-122``) and raise ``ValueError``. With
``enable_minibatching`` the features (and weights) are a sequence of
minibatches, each preprocessed on its own and packed into the minibatching
layout of ``_pack_partitions_to_csr`` (``:190-284``). The returned buffers
are torch CUDA tensors.
"""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from jax_tpu_embedding.sparsecore.utils import utils


def _resolve_feature_input_ndim(features) -> int:
  if isinstance(features, np.ndarray):
    return features.ndim
  t = _native.torch()
  if isinstance(features, t.Tensor):
    return features.dim()
  try:
    return np.asarray(features, dtype=object).ndim
  except ValueError:
    return 1


def _global_device_count(mesh) -> int:
  """Devices of a mesh-like argument: an object with a ``devices`` array
  (jax.sharding.Mesh), a sequence of devices, or a count."""
  if isinstance(mesh, (int, np.integer)):
    return int(mesh)
  devices = getattr(mesh, "devices", mesh)
  return int(np.size(np.asarray(devices, dtype=object)))


def _as_samples(features, weights):
  """Per-sample id and weight arrays (ragged object arrays)."""
  n = len(features)
  ids = np.empty(n, dtype=object)
  wts = np.empty(n, dtype=object)
  t = _native.torch()
  for i in range(n):
    f = features[i]
    w = weights[i] if weights is not None else None
    if isinstance(f, t.Tensor):
      f = f.cpu().numpy()
    if isinstance(w, t.Tensor):
      w = w.cpu().numpy()
    f = np.asarray(f, dtype=np.int32).reshape(-1)
    w = (np.ones(f.shape, np.float32) if w is None else
         np.asarray(w, dtype=np.float32).reshape(-1))
    if f.shape != w.shape:
      raise ValueError(
          f"features and features_weights of sample {i} have different "
          f"lengths: {f.shape[0]} and {w.shape[0]}.")
    ids[i] = f
    wts[i] = w
  return ids, wts


def single_feature_spec(batch: int, max_id: int, max_ids_per_partition: int,
                        max_unique_ids_per_partition: int,
                        global_device_count: int, num_sc: int):
  """The one-feature, one-table stack (sum combiner) the reference module's
  partitioning corresponds to, prepared for `global_device_count` devices of
  `num_sc` SparseCores. Any table height that holds every id works: column
  ids do not depend on it (partition = id % num_scs, embedding id =
  id // num_scs)."""
  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top

  num_scs = num_sc * global_device_count
  vocab = (max_id + 1 + 8 * num_scs - 1) // (8 * num_scs) * (8 * num_scs)
  table = embedding_spec.TableSpec(
      name="table", vocabulary_size=vocab, embedding_dim=8,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.0), combiner="sum",
      max_ids_per_partition=max(max_ids_per_partition, 1),
      max_unique_ids_per_partition=max(max_unique_ids_per_partition, 1))
  feature = embedding_spec.FeatureSpec(
      name="feature", table_spec=table, input_shape=[batch, 1],
      output_shape=[batch, 8])
  embedding.prepare_feature_specs_for_training(
      [feature], global_device_count=global_device_count,
      num_sc_per_device=num_sc)
  return feature


def preprocess_sparse_dense_matmul_input(
    features, features_weights, mesh, *, max_ids_per_partition: int,
    max_unique_ids_per_partition: int, num_sc_per_device: int = -1,
    sharding_strategy: str = "MOD", enable_minibatching: bool = False):
  """Returns (row_pointers, embedding_ids, sample_ids, gains) for one feature
  batch (or, with `enable_minibatching`, a sequence of minibatches) on one
  device (reference ``input_preprocessing.py:290-383``)."""
  if max_ids_per_partition <= 0:
    raise ValueError(
        f"max_ids_per_partition must be positive, got {max_ids_per_partition}.")
  ndim = _resolve_feature_input_ndim(features)
  if not enable_minibatching and ndim not in (1, 2):
    raise ValueError(f"features must be 1D or 2D, got {ndim}D.")
  if features_weights is not None and len(features) != len(features_weights):
    raise ValueError("features and features_weights must have the same length.")
  if sharding_strategy != "MOD":
    raise ValueError("Currently only MOD sharding strategy is supported")
  global_device_count = _global_device_count(mesh)
  if global_device_count <= 0:
    raise ValueError("global_device_count must be positive.")
  num_sc = (num_sc_per_device if num_sc_per_device > 0 else
            utils.num_sparsecores_per_device())
  if enable_minibatching:
    t = _native.torch()
    if isinstance(features, (np.ndarray, t.Tensor)) or not hasattr(
        features, "__len__"):
      raise ValueError("When enable_minibatching is True, features must be a "
                       "sequence of batches.")
    weights = (features_weights if features_weights is not None else
               [None] * len(features))
    parts = [
        _preprocess_one(f, w, max_ids_per_partition,
                        max_unique_ids_per_partition, global_device_count,
                        num_sc) for f, w in zip(features, weights)
    ]
    return _pack_minibatches(parts, num_sc, num_sc * global_device_count)
  return _preprocess_one(features, features_weights, max_ids_per_partition,
                         max_unique_ids_per_partition, global_device_count,
                         num_sc)


def _pack_minibatches(parts, num_sc: int, num_scs: int):
  """The minibatching layout of _pack_partitions_to_csr (reference
  input_preprocessing.py:190-284): for each local SC (starting at the
  aligned end of the one before) and each minibatch, the partitions' entries
  at positions in the whole buffer, row pointers at their ends, each
  partition starting 8-aligned, max(NS, 8) row pointers per minibatch; every
  other position holds the padding (INT_MAX, INT_MAX, NaN). The entries are
  copied on the device; only the minibatches' row pointers are read back."""
  t = _native.torch()
  dev = _native.device()
  per_mb = int(parts[0][1].numel())
  total = per_mb * len(parts)
  eid = t.full((total,), np.iinfo(np.int32).max, dtype=t.int32, device=dev)
  sid = t.full((total,), np.iinfo(np.int32).max, dtype=t.int32, device=dev)
  gains = t.full((total,), float("nan"), dtype=t.float32, device=dev)
  rps_host = [p[0].cpu().numpy() for p in parts]
  rpb = max(num_scs, 8)
  rp = []
  coo = 0
  for s in range(num_sc):
    coo = -(-coo // 8) * 8
    for m, (_, e, si, g) in enumerate(parts):
      seg = int(e.numel()) // num_sc
      rpm = rps_host[m][s * (len(rps_host[m]) // num_sc):]
      start = 0
      for p in range(num_scs):
        end = int(rpm[p])
        n = end - start
        if n > 0:
          src = slice(s * seg + start, s * seg + end)
          eid[coo:coo + n] = e[src]
          sid[coo:coo + n] = si[src]
          gains[coo:coo + n] = g[src]
          coo += n
        rp.append(coo)
        coo = -(-coo // 8) * 8
        start = -(-end // 8) * 8
      rp.extend([coo] * (rpb - num_scs))
  return (t.tensor(np.array(rp, np.int32), device=dev), eid, sid, gains)


def _preprocess_one(features, features_weights, max_ids_per_partition,
                    max_unique_ids_per_partition, global_device_count, num_sc):
  """One batch through the stacked pipeline, checked against the limits."""
  ids, wts = _as_samples(features, features_weights)
  batch = len(ids)
  max_id = max((int(r.max()) for r in ids if r.size), default=0)
  if any(r.size and int(r.min()) < 0 for r in ids):
    raise ValueError("ids must be non-negative.")
  feature = single_feature_spec(batch, max_id, max_ids_per_partition,
                                max_unique_ids_per_partition,
                                global_device_count, num_sc)
  table = feature.table_spec
  # Dropping is enabled so that an over-limit batch still yields its
  # observed counts; such a batch raises below.
  rp, eid, sid, gains, _, stats = (
      pybind_input_preprocessing.preprocess_sparse_dense_matmul_input(
          [ids], [wts], [feature], 1, global_device_count,
          num_sc_per_device=num_sc, allow_id_dropping=True))
  name = table.stacked_table_spec.stack_name
  observed_ids = int(np.max(stats.max_ids_per_partition[name]))
  observed_unique = int(np.max(stats.max_unique_ids_per_partition[name]))
  if observed_ids > max_ids_per_partition:
    raise ValueError(f"Partition has too many ids. {observed_ids} >"
                     f" {max_ids_per_partition}.")
  if observed_unique > max_unique_ids_per_partition:
    raise ValueError(f"Partition has too many unique ids. {observed_unique} >"
                     f" {max_unique_ids_per_partition}.")
  return rp[name], eid[name], sid[name], gains[name]
