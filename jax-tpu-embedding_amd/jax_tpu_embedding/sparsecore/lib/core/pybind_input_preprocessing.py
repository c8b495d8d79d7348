"""GPU preprocessing with the interface of the reference's pybind module.

Mirrors ``lib/core/pybind_input_preprocessing.cc`` (functions bound at
:291-330, stubs in ``pybind_input_preprocessing.pyi:38-86``): same function
names, argument meaning, output tuple and exceptions (``ValueError`` for
invalid arguments, ``RuntimeError`` where the reference aborts). The work runs
on the GPU through ``scemb_preprocess_stacked_table``; outputs are torch CUDA
tensors (flattened unless ``has_leading_dimension``), stats are numpy.

Minibatching (``enable_minibatching=True``) is single-host: the passes of
``PreprocessSparseDenseMatmulInput`` (input_preprocessing.cc:852-929) run as
one library call per pass and stack, with the OR of the stacks' splits taken
here (the reference's all-reduce across hosts is not part of this path).
"""

from __future__ import annotations

import ctypes
import dataclasses
import enum

import numpy as np

from jax_tpu_embedding.sparsecore import _native

_COMBINERS = {"sum": 0, "mean": 1, "sqrtn": 2}
# PreprocessOptions.flags of every call (_native.PREPROCESS_*); 0 lets the
# library pick the grouping route.
PREPROCESS_FLAGS = 0


class ShardingStrategy(enum.IntEnum):
  MOD = 1


class AllReduceInterface:  # pylint: disable=too-few-public-methods
  """Placeholder type: cross-host minibatching is not part of this path (one
  host decides alone, input_preprocessing.cc:535-537, :581-583)."""


class SparseDenseMatmulInputStats:
  """Stats of one preprocessing call (input_preprocessing.h:30-43)."""

  def __init__(self):
    self.max_ids_per_partition = {}
    self.max_unique_ids_per_partition = {}
    self.required_buffer_sizes = {}
    self.dropped_id_count = {}
    # No reference counterpart: grouped CSR entries per stacked table (an
    # upper bound on the valid entries; lets the lookup pick its kernels).
    self.num_entries = {}

  def TotalDroppedIdCount(self) -> int:  # pylint: disable=invalid-name
    return int(sum(self.dropped_id_count.values()))


@dataclasses.dataclass
class FeatureMetadataInStack:
  """One feature of a stacked table (input_preprocessing_util.h:524-571)."""

  name: str
  feature_index: int
  max_ids_per_partition: int
  max_unique_ids_per_partition: int
  row_offset: int
  col_offset: int
  col_shift: int
  batch_size: int
  suggested_coo_buffer_size_per_device: int | None
  row_combiner: str
  max_col_id: int
  stack_vocab_size: int


def get_stacked_table_metadata(feature_specs):
  """GetStackedTableMetadata (pybind_input_preprocessing.cc:55-122)."""
  out: dict[str, list[FeatureMetadataInStack]] = {}
  for i, fs in enumerate(feature_specs):
    tr = fs._id_transformation  # pylint: disable=protected-access
    table_spec = fs.table_spec
    stacked = table_spec.stacked_table_spec
    if stacked is None:
      raise ValueError(f"stacked_table_spec is none for table {table_spec.name}")
    stack_name = table_spec.setting_in_stack.stack_name
    row_offset = col_offset = col_shift = 0
    if tr is not None:
      row_offset, col_offset, col_shift = (int(tr.row_offset),
                                           int(tr.col_offset),
                                           int(tr.col_shift))
    out.setdefault(stack_name, []).append(
        FeatureMetadataInStack(
            name=fs.name,
            feature_index=i,
            max_ids_per_partition=int(stacked.max_ids_per_partition),
            max_unique_ids_per_partition=int(
                stacked.max_unique_ids_per_partition),
            row_offset=row_offset,
            col_offset=col_offset,
            col_shift=col_shift,
            batch_size=int(fs.input_shape[0]),
            suggested_coo_buffer_size_per_device=(
                stacked.suggested_coo_buffer_size_per_device),
            row_combiner=stacked.combiner,
            max_col_id=int(table_spec.vocabulary_size),
            stack_vocab_size=int(stacked.stack_vocab_size)))
  for metas in out.values():
    metas.sort(key=lambda m: m.row_offset)
  return out


# ---------------------------------------------------------------------------
# Size helpers (pybind_input_preprocessing.cc:203-262, bound at :311-320).
# ---------------------------------------------------------------------------


def compute_row_pointers_size_per_device(global_device_count: int,
                                         num_sc_per_device: int,
                                         enable_minibatching: bool = False):
  return int(_native.load_library().scemb_compute_row_pointers_size_per_device(
      global_device_count, num_sc_per_device, int(bool(enable_minibatching))))


def compute_theoretical_max_coo_buffer_size(max_ids_per_partition: int,
                                            global_device_count: int,
                                            num_sc_per_device: int,
                                            enable_minibatching: bool = False):
  return int(
      _native.load_library().scemb_compute_theoretical_max_coo_buffer_size(
          max_ids_per_partition, global_device_count, num_sc_per_device,
          int(bool(enable_minibatching))))


def _coo_buffer_size(meta: FeatureMetadataInStack, global_device_count,
                     num_sc_per_device, enable_minibatching=False) -> int:
  v = _native.load_library().scemb_compute_coo_buffer_size_per_device(
      meta.max_ids_per_partition,
      meta.suggested_coo_buffer_size_per_device or 0, global_device_count,
      num_sc_per_device, int(bool(enable_minibatching)))
  if v < 0:
    raise RuntimeError(
        "Suggested Coo Buffer Size is larger than the theoretical max for "
        f"table {meta.name}. Adjust the suggested size or the "
        "max_ids_per_partition values.")
  if v >= 2**31 - 1:
    raise RuntimeError(f"Computed Coo Buffer Size ({v}) for table "
                       f"{meta.name} is out of the valid range (0, INT_MAX).")
  return int(v)


def compute_coo_buffer_size_per_device(feature_specs, global_device_count: int,
                                       num_sc_per_device: int,
                                       enable_minibatching: bool = False):
  stacks = get_stacked_table_metadata(list(feature_specs))
  return {
      name: _coo_buffer_size(metas[0], global_device_count, num_sc_per_device,
                             enable_minibatching)
      for name, metas in stacks.items()
  }


# ---------------------------------------------------------------------------
# Input conversion.
# ---------------------------------------------------------------------------


@dataclasses.dataclass
class _DeviceFeature:
  ids: object
  weights: object | None
  splits: object | None
  splits_host: np.ndarray | None
  num_rows: int
  nnz: int
  valency: int
  max_id: int | None  # known when the input came from host memory
  max_row_length: int | None = None  # most ids of one row (None: not known)
  # Device buffers that staged fields live in once they are addresses: held
  # as long as the feature (the pending call keeps its features until its
  # stats are collected, after every kernel that reads them).
  keep: list | None = None

  @property
  def one_id_per_row(self) -> bool:
    """No row holds two ids. False for ragged rows whose longest length is
    not known yet (row splits staged but not checked)."""
    if self.splits_host is None:
      return self.valency <= 1
    return self.max_row_length is not None and self.max_row_length <= 1


def _to_device_feature(feature, weights, uploads=None,
                       dev=None) -> _DeviceFeature:
  """One feature's ids, weights and row splits as device tensors. With
  `uploads` (a _native.HostUploads), host arrays are staged there instead of
  copied one by one: the fields hold handles until _resolve_feature runs
  after uploads.flush(). `dev`: the current device, when the caller has it."""
  t = _native.require_gpu()
  if dev is None:
    dev = _native.device()

  def on_device(x, dtype):
    if isinstance(x, t.Tensor):
      # Already where it goes (the common case for inputs kept in HBM): the
      # tensor itself, whose contiguous elements are the flat layout the
      # library reads (a view would cost host time and change nothing).
      if (x.is_cuda and x.dtype == dtype and x.get_device() == dev.index and
          x.is_contiguous()):
        return x
      return _native.as_device_tensor(x.reshape(-1), dtype, dev)
    if uploads is None:
      return _native.as_device_tensor(x, dtype, dev)
    return uploads.add(x, dtype)

  if isinstance(feature, t.Tensor):
    nd = feature.dim()
    if nd == 1:
      rows, cols = int(feature.shape[0]), 1
    elif nd == 2:
      rows, cols = int(feature.shape[0]), int(feature.shape[1])
    else:
      raise ValueError("Only 1D and 2D inputs are supported.")
    ids = on_device(feature, t.int32)
    w = None
    if weights is not None:
      w = on_device(
          weights if isinstance(weights, t.Tensor) else
          np.asarray(weights, np.float32).reshape(-1), t.float32)
    return _DeviceFeature(ids, w, None, None, rows, rows * cols, cols, None)
  if hasattr(feature, "values") and hasattr(feature, "row_splits"):
    # Ragged tensor (tf.RaggedTensor-like: flat values + row splits), the
    # RaggedTensorInputBatch input of ragged_tensor_input_batch.h:68-127.
    vals = feature.values
    splits = np.ascontiguousarray(feature.row_splits,
                                  dtype=np.int64).reshape(-1)
    if isinstance(vals, t.Tensor):
      vals = vals.reshape(-1)
    else:
      vals = np.ascontiguousarray(np.asarray(vals), dtype=np.int32).reshape(-1)
    if uploads is not None:
      # Checked while staged (flush); the longest row comes back then.
      splits_dev = uploads.add_row_splits(splits, int(vals.shape[0]))
      max_len = None
    else:
      max_len = _check_row_splits(splits, int(vals.shape[0]))
      splits_dev = on_device(splits, t.int64)
    w = None
    if weights is not None:
      wv = getattr(weights, "values", weights)
      wv = (wv.reshape(-1) if isinstance(wv, t.Tensor) else
            np.asarray(wv, np.float32).reshape(-1))
      if wv.shape[0] != vals.shape[0]:
        raise ValueError("Batch size mismatch for features and weights.")
      w = on_device(wv, t.float32)
    ids = on_device(vals, t.int32)
    max_id = None
    if not isinstance(vals, t.Tensor) and vals.size:
      max_id = int(vals.max())
    return _DeviceFeature(ids, w, splits_dev, splits, splits.size - 1,
                          int(splits[-1]), 0, max_id, max_len)
  arr = feature if isinstance(feature, np.ndarray) else np.asarray(
      feature, dtype=object)
  if arr.dtype != object and arr.ndim == 2:
    ids_np = np.ascontiguousarray(arr, dtype=np.int32).reshape(-1)
    w_np = None
    if weights is not None:
      w_np = np.ascontiguousarray(np.asarray(weights, dtype=np.float32)
                                  ).reshape(-1)
      if w_np.shape != ids_np.shape:
        raise ValueError("Batch size mismatch for features and weights.")
    b, k = arr.shape
    max_id = int(ids_np.max()) if ids_np.size else None
    return _DeviceFeature(
        on_device(ids_np, t.int32),
        None if w_np is None else on_device(w_np, t.float32),
        None, None, b, b * k, k, max_id)
  if arr.dtype != object and arr.ndim == 1:
    # One id per sample.
    return _to_device_feature(arr.reshape(-1, 1),
                              None if weights is None else
                              np.asarray(weights, np.float32).reshape(-1, 1),
                              uploads)
  if arr.ndim != 1:
    raise ValueError("Only 1D and 2D numpy arrays supported as inputs.")
  rows = [np.asarray(r).reshape(-1) for r in arr]
  lens = np.fromiter((len(r) for r in rows), dtype=np.int64, count=len(rows))
  splits = np.zeros(len(rows) + 1, np.int64)
  np.cumsum(lens, out=splits[1:])
  ids_np = (np.concatenate(rows).astype(np.int32) if splits[-1] else
            np.zeros(0, np.int32))
  w_np = None
  if weights is not None:
    wrows = [np.asarray(x, np.float32).reshape(-1) for x in weights]
    if len(wrows) != len(rows) or any(
        len(a) != len(b) for a, b in zip(wrows, rows)):
      raise ValueError("Batch size mismatch for features and weights.")
    w_np = (np.concatenate(wrows) if splits[-1] else np.zeros(0, np.float32))
  max_id = int(ids_np.max()) if ids_np.size else None
  return _DeviceFeature(
      on_device(ids_np, t.int32),
      None if w_np is None else on_device(w_np, t.float32),
      on_device(splits, t.int64), splits, len(rows),
      int(splits[-1]), 0, max_id, int(lens.max()) if lens.size else 0)


def _check_row_splits(splits: np.ndarray, nnz: int) -> int:
  """The most ids of one row; raises ValueError unless the row splits start
  at 0, do not decrease and end at `nnz` (one pass in the library)."""
  if splits.size == 0:
    raise ValueError(_native.ROW_SPLITS_MESSAGE)
  out = ctypes.c_int64(0)
  rc = _native.load_library().scemb_check_row_splits(
      splits.ctypes.data, splits.size - 1, nnz, ctypes.byref(out))
  if rc != 0:
    raise ValueError(_native.ROW_SPLITS_MESSAGE)
  return int(out.value)


def _resolve_feature(f: _DeviceFeature) -> _DeviceFeature:
  """Staged fields become device addresses (_native.ptr takes both); the
  rows' longest length comes from the staging check."""
  handle = _native.HostUploads.Handle
  if not (isinstance(f.ids, handle) or isinstance(f.weights, handle) or
          isinstance(f.splits, handle)):
    return f  # nothing was staged: device tensors (or None) as they are
  if getattr(f.splits, "max_row_length", None) is not None:
    f.max_row_length = f.splits.max_row_length
  f.keep = [h.base for h in (f.ids, f.weights, f.splits)
            if isinstance(h, _native.HostUploads.Handle)]
  f.ids = _native.HostUploads.resolve_address(f.ids)
  f.weights = _native.HostUploads.resolve_address(f.weights)
  f.splits = _native.HostUploads.resolve_address(f.splits)
  return f


class _StackCall:
  """One stack's library call, prepared by _prepare_stack: its ctypes
  arguments (held until the call) and the workspace it needs."""
  __slots__ = ("structs", "num_features", "opts", "out", "need")

  def __init__(self, structs, num_features, opts, out, need):
    self.structs, self.num_features = structs, num_features
    self.opts, self.out, self.need = opts, out, need


def _preprocess_stack(feats, metas, *, stream=None, **kwargs):
  """Enqueues one stacked table (one minibatching pass of it with
  `enable_minibatching`); returns what _prepare_stack does. `stream` (may be
  None): the stream to enqueue on instead of the current one; the outputs
  are still allocated on the current stream, which the caller makes wait for
  `stream` before it uses them."""
  call, result = _prepare_stack(feats, metas, **kwargs)
  lib = _native.load_library()
  # The workspace belongs to the stream the work is enqueued on.
  ws = _native.WORKSPACE.get(call.need, stream)
  _native.check(lib.scemb_preprocess_stacked_table(
      call.structs, call.num_features, ctypes.byref(call.opts),
      ctypes.byref(call.out), _native.ptr(ws), ws.numel(),
      stream.cuda_stream if stream is not None else _native.stream_handle()))
  return result


def _preprocess_stacks(calls):
  """Enqueues prepared stacks with one library call on the current stream
  (scemb_preprocess_stacked_tables: one launch per stage for the stacks that
  merge duplicates at extraction), each with its slice of one workspace."""
  if not calls:
    return
  sizes = [-(-c.need // 256) * 256 for c in calls]
  ws = _native.WORKSPACE.get(sum(sizes))
  base = _native.ptr(ws)
  jobs = (_native.PreprocessJob * len(calls))()
  pos = 0
  for job, c, size in zip(jobs, calls, sizes):
    job.features = c.structs.address
    job.num_features = c.num_features
    job.options = ctypes.addressof(c.opts)
    job.outputs = ctypes.addressof(c.out)
    job.workspace = base + pos
    job.workspace_bytes = size
    pos += size
  _native.check(_native.load_library().scemb_preprocess_stacked_tables(
      jobs, len(calls), _native.stream_handle()))


class _StackPlan:
  """What one stack's library call needs besides its outputs (_plan_stack):
  the ctypes options and features (held until the call), the workspace
  bytes, the COO buffer size per device and the stats layout."""
  __slots__ = ("structs", "num_features", "opts", "need", "coo", "L", "S",
               "ns", "off")


def _plan_stack(feats, metas, *, local_device_count, global_device_count,
                num_sc_per_device, allow_id_dropping, has_weights,
                build_view=False, enable_minibatching=False,
                minibatching_pass=0, minibatching_split=0) -> _StackPlan:
  lib = _native.load_library()
  ns = num_sc_per_device * global_device_count
  c = _coo_buffer_size(metas[0], global_device_count, num_sc_per_device,
                       enable_minibatching)
  bound = max(m.stack_vocab_size for m in metas)
  for f, m in zip(feats, metas):
    if f.max_id is not None:
      bound = max(bound, m.col_offset + f.max_id + ns + 1)
  plan = _StackPlan()
  plan.opts = _native.PreprocessOptions(
      local_device_count, global_device_count, num_sc_per_device,
      _COMBINERS.get(metas[0].row_combiner, 0),
      metas[0].max_ids_per_partition, metas[0].max_unique_ids_per_partition,
      int(bool(allow_id_dropping)), int(bool(has_weights)), c, bound,
      int(bool(build_view)), int(bool(enable_minibatching)),
      metas[0].stack_vocab_size // global_device_count,
      int(minibatching_pass), PREPROCESS_FLAGS, int(minibatching_split))
  plan.structs = _native.feature_structs(
      [(_native.ptr(f.ids), _native.ptr(f.weights), _native.ptr(f.splits),
        0 if f.splits_host is None else f.splits_host.ctypes.data,
        f.num_rows, f.nnz, f.valency, m.row_offset, m.col_offset, m.col_shift,
        f.max_row_length or 0) for f, m in zip(feats, metas)])
  plan.num_features = len(feats)
  plan.need = lib.scemb_preprocess_workspace_size(plan.structs, len(feats),
                                                  ctypes.byref(plan.opts))
  if plan.need == 0:
    _native.check(_native.SCEMB_ERR_INVALID_ARGUMENT)
  plan.coo, plan.L, plan.S, plan.ns = c, local_device_count, num_sc_per_device, ns
  # The stats block's int64 counters follow the per-partition stats
  # (scemb_preprocess_stats_counters_offset).
  stats = 2 * plan.L * ns + plan.L * plan.S
  plan.off = stats + stats % 2
  return plan


def _output_words(plan, enable_minibatching, build_view, outputs=True):
  """int32 words of a stack's outputs, in order: row pointers, ids, samples,
  gains (unless `outputs` is false), then view keys and entries."""
  L, S, c = plan.L, plan.S, plan.coo
  parts = []
  if outputs:
    parts += [L * S * max(plan.ns, 8) *
              (_native.MAX_MINIBATCHES if enable_minibatching else 1),
              L * c, L * c, L * c]
  if build_view:
    parts += [c, 2 * c]
  return parts


def _prepare_stack(feats, metas, *, local_device_count, global_device_count,
                   num_sc_per_device, allow_id_dropping, has_weights,
                   build_view=False, enable_minibatching=False,
                   minibatching_pass=0, minibatching_split=0, outputs=None,
                   view_outputs=None, stats_out=None):
  """The library call of one stacked table (one minibatching pass of it with
  `enable_minibatching`), not yet made, and its outputs: (call, (rp, eid,
  sid, gains, stats on the device, (L, S, NS, counters offset), view)) where
  view is the (keys, entries) pair of the CSR's sample view when
  `build_view`, else None. `outputs` / `view_outputs`: the (rp, eid, sid,
  gains) / view of an earlier pass to write into. `stats_out`: an int32
  device tensor of _stats_words(...) slots to hold the stats (else one is
  allocated). The outputs are allocated on the current stream."""
  t = _native.require_gpu()
  dev = _native.device()
  plan = _plan_stack(
      feats, metas, local_device_count=local_device_count,
      global_device_count=global_device_count,
      num_sc_per_device=num_sc_per_device,
      allow_id_dropping=allow_id_dropping, has_weights=has_weights,
      build_view=build_view, enable_minibatching=enable_minibatching,
      minibatching_pass=minibatching_pass,
      minibatching_split=minibatching_split)
  # Outputs not given come out of one allocation (int32 words, each part
  # 256-byte aligned).
  parts = _output_words(plan, enable_minibatching,
                        build_view and not view_outputs, outputs is None)
  if parts:
    sizes = [-(-n // 64) * 64 for n in parts]
    block = t.empty(max(sum(sizes), 1), dtype=t.int32, device=dev)
    carved, pos = [], 0
    for n, size in zip(parts, sizes):
      carved.append(block[pos:pos + n])
      pos += size
  if outputs is not None:
    rp, eid, sid, gains = outputs
  else:
    rp, eid, sid, gains = carved[:4]
    gains = gains.view(t.float32)
    carved = carved[4:]
  nstats = plan.off + 2 * _NUM_COUNTERS
  # The library initialises the whole stats block.
  if stats_out is not None:
    if int(stats_out.numel()) < nstats:
      raise ValueError("stats buffer too small")
    stats = stats_out
  else:
    stats = t.empty(nstats + 2, dtype=t.int32, device=dev)
  view = None
  if build_view:
    view = view_outputs or (carved[0], carved[1].view(t.int64))
  out = _native.PreprocessOutput(
      _native.ptr(rp), _native.ptr(eid), _native.ptr(sid), _native.ptr(gains),
      _native.ptr(stats), None if view is None else _native.ptr(view[0]),
      None if view is None else _native.ptr(view[1]))
  # The stats stay on the device until every stack has been enqueued.
  return (_StackCall(plan.structs, plan.num_features, plan.opts, out,
                     plan.need),
          (rp, eid, sid, gains, stats, (plan.L, plan.S, plan.ns, plan.off),
           view))


def _stats_words(local_device_count, global_device_count, num_sc_per_device):
  """int32 slots of one stack's stats block (scemb_preprocess_stats_size:
  the per-partition stats rounded up to an even count, then six int64
  counters), plus two so that consecutive blocks keep the counters 8-byte
  aligned."""
  L, S = local_device_count, num_sc_per_device
  ns = S * global_device_count
  stats = 2 * L * ns + L * S
  return stats + stats % 2 + 2 * _NUM_COUNTERS + 2


def preprocess_sparse_dense_matmul_input(
    features,
    feature_weights,
    feature_specs,
    local_device_count: int,
    global_device_count: int,
    *,
    num_sc_per_device: int,
    sharding_strategy=ShardingStrategy.MOD,
    has_leading_dimension: bool = False,
    allow_id_dropping: bool = False,
    batch_number: int = 0,
    enable_minibatching: bool = False,
    all_reduce_interface=None,
):
  """PyNumpyPreprocessSparseDenseMatmulInput (pybind_input_preprocessing.cc:
  190-216 and :124-188) on the GPU.

  Returns (row_pointers, embedding_ids, sample_ids, gains, num_minibatches,
  stats): four dicts keyed by stacked-table name, the minibatch count and a
  SparseDenseMatmulInputStats.
  """
  del batch_number, all_reduce_interface
  features, feature_weights, feature_specs = check_arguments(
      features, feature_weights, feature_specs, sharding_strategy,
      enable_minibatching, local_device_count=local_device_count,
      global_device_count=global_device_count,
      num_sc_per_device=num_sc_per_device)
  rps, eids, sids, gns, pending = enqueue_preprocessing(
      features, feature_weights, feature_specs, local_device_count,
      global_device_count, num_sc_per_device=num_sc_per_device,
      has_leading_dimension=has_leading_dimension,
      allow_id_dropping=allow_id_dropping,
      enable_minibatching=enable_minibatching)
  return (rps, eids, sids, gns, pending.num_minibatches,
          collect_stats(pending))


def check_arguments(features, feature_weights, feature_specs,
                    sharding_strategy, enable_minibatching: bool, *,
                    local_device_count: int, global_device_count: int,
                    num_sc_per_device: int):
  """Argument checks of the preprocessing entry, before any device work;
  returns the inputs as lists. The option checks and their messages are
  PreprocessSparseDenseMatmulInputOptions::Validate
  (input_preprocessing_util.cc:490-522), then the empty-input check
  (input_preprocessing.cc:815-817); the library repeats them."""
  del enable_minibatching  # every combination is accepted
  if int(sharding_strategy) != int(ShardingStrategy.MOD):
    raise ValueError("Only mod sharding is supported for now.")
  if local_device_count <= 0:
    raise ValueError("local_device_count must be greater than 0, but got "
                     f"{local_device_count}")
  if global_device_count <= 0:
    raise ValueError("global_device_count must be greater than 0, but got "
                     f"{global_device_count}")
  if global_device_count < local_device_count:
    raise ValueError(
        "global_device_count must be greater than or equal to "
        f"local_device_count, but got {global_device_count} vs "
        f"{local_device_count}")
  if num_sc_per_device <= 0:
    raise ValueError("num_sc_per_device must be greater than 0, but got "
                     f"{num_sc_per_device}")
  num_scs = num_sc_per_device * global_device_count
  if num_scs & (num_scs - 1):
    raise ValueError(f"Total number of SparseCores ({num_scs}) must be a "
                     "power of 2.")
  features = list(features)
  feature_specs = list(feature_specs)
  if feature_weights is not None:
    feature_weights = list(feature_weights)
    if len(feature_weights) != len(features):
      raise ValueError("features and feature_weights must have equal length")
  if len(features) != len(feature_specs):
    raise ValueError("features and feature_specs must have equal length")
  if not features:
    raise ValueError("input_batches cannot be empty.")
  return features, feature_weights, feature_specs


class PendingStats(list):
  """Per stack (name, stats on the device, L, S, NS, counters offset,
  features) of the enqueued first pass, plus what minibatching decided:
  `num_minibatches` and, per stack, the stats of the pass that wrote the
  final CSR when it was not the first (its dropped ids count)."""

  def __init__(self):
    super().__init__()
    self.num_minibatches = 1
    self.final_pass_stats = {}
    self.stats_buffer = None  # the stacks' first-pass stats, one after another
    # Without minibatching: the stats block's copy into pinned host memory,
    # enqueued behind the preprocessing on its stream, and the event that
    # marks it done.
    self.host_stats = None
    self.host_stats_ready = None


def _to_host(tensors) -> np.ndarray:
  """The int32 device tensors, one after another, in one pinned host
  buffer: asynchronous copies on the current stream, then one wait."""
  t = _native.torch()
  host = t.empty(sum(int(x.numel()) for x in tensors), dtype=t.int32,
                 pin_memory=True)
  pos = 0
  for x in tensors:
    n = int(x.numel())
    host[pos:pos + n].copy_(x, non_blocking=True)
    pos += n
  t.cuda.current_stream().synchronize()
  return host.numpy()


def _read_counters(entries, buffer=None):
  """One wait: the int64 counters of each (stats tensor, offset); `buffer`
  (may be None): one device tensor holding the stats tensors in order."""
  host = _to_host([buffer] if buffer is not None else [e[0] for e in entries])
  out, pos = [], 0
  for stats_dev, off in entries:
    chunk = host[pos:pos + stats_dev.numel()]
    pos += stats_dev.numel()
    out.append(chunk[off:off + 2 * _NUM_COUNTERS].copy().view(np.int64))
  return out


_NUM_COUNTERS = 6


def _raise_on_counters(name, counters):
  if counters[2] > 0:
    raise ValueError(
        f"{int(counters[2])} embedding ids of stacked table {name} are "
        "negative or beyond the stacked vocabulary.")
  if counters[1] > 0:
    raise RuntimeError(
        f"Observed max ids per partition for table: {name} is greater than "
        "the set max ids per partition. Use `allow_id_dropping` or increase "
        "the `max_ids_per_partition`. You could also try to reduce the "
        "batch size.")


def _minibatching_passes(pending, jobs, csr, views):
  """Runs the rest of input_preprocessing.cc:852-929 after every stack's
  first pass: if one of them exceeds a limit, the OR of the stacks' splits
  and the minibatched fill of every stack. The first pass already counted
  its runs per bucket when a limit was exceeded, so its counter 5 is the
  bucket pass's split (the library's pass 1 gives the same; the tests
  compare them). Waits for the device once."""
  first = _read_counters([(p[1], p[5]) for p in pending],
                         pending.stats_buffer)
  for p, c in zip(pending, first):
    _raise_on_counters(p[0], c)
  if not any(c[4] for c in first):
    return
  split = 0
  for c in first:
    split |= int(np.uint64(c[5]))
  for name, kwargs in jobs:
    out = _preprocess_stack(**kwargs, minibatching_pass=2,
                            minibatching_split=split, outputs=csr[name],
                            build_view=name in views,
                            view_outputs=views.get(name))
    pending.final_pass_stats[name] = (out[4], out[5][3])
  pending.num_minibatches = bin(split).count("1") + 1


def enqueue_preprocessing(features, feature_weights, feature_specs,
                          local_device_count: int, global_device_count: int,
                          *, num_sc_per_device: int,
                          has_leading_dimension: bool = False,
                          allow_id_dropping: bool = False,
                          sample_views: dict | None = None,
                          enable_minibatching: bool = False):
  """Enqueues the preprocessing of every stack on the current stream without
  waiting for it. Returns the CSR dicts and the pending stats, which
  collect_stats turns into a SparseDenseMatmulInputStats (one wait). With a
  `sample_views` dict (one local and one global device only), each stack's
  sample view (keys, entries) is built along and stored there. With
  `enable_minibatching` the minibatching passes run here (they wait for the
  device) and `pending.num_minibatches` holds the outcome; a sample view is
  rebuilt by the pass that writes the final CSR."""
  stacks = get_stacked_table_metadata(feature_specs)
  rps, eids, sids, gns = {}, {}, {}, {}
  pending = PendingStats()
  jobs, flat = [], {}
  build_view = (sample_views is not None and local_device_count == 1 and
                global_device_count == 1)
  # Host inputs of every stack go to the device in one copy.
  uploads = _native.HostUploads()
  dev = _native.device()
  stack_feats = {
      name: [
          _to_device_feature(
              features[m.feature_index],
              None if feature_weights is None else
              feature_weights[m.feature_index], uploads, dev) for m in metas
      ] for name, metas in stacks.items()
  }
  uploads.flush()
  # The stats of every stack's first pass share one device buffer, so that
  # collect_stats reads them back with one copy.
  words = _stats_words(local_device_count, global_device_count,
                       num_sc_per_device)
  t = _native.torch()
  pending.stats_buffer = t.empty(words * len(stacks), dtype=t.int32,
                                 device=_native.device())
  # Every stack goes to the library in one call on the current stream, which
  # runs each stage of the stacks that merge duplicates at extraction as one
  # launch for all of them (the kernels of one stage then fill the device
  # together). The call takes the outputs' addresses in one block for all
  # stacks; their tensors are made while the device works.
  plans, layout, total = [], [], 0
  for name, metas in stacks.items():
    feats = [_resolve_feature(f) for f in stack_feats[name]]
    kwargs = dict(feats=feats, metas=metas,
                  local_device_count=local_device_count,
                  global_device_count=global_device_count,
                  num_sc_per_device=num_sc_per_device,
                  allow_id_dropping=allow_id_dropping,
                  has_weights=feature_weights is not None,
                  enable_minibatching=enable_minibatching)
    plan = _plan_stack(**kwargs, build_view=build_view)
    if plan.off + 2 * _NUM_COUNTERS > words:
      raise ValueError("stats buffer too small")
    parts = _output_words(plan, enable_minibatching, build_view)
    offs = []
    for n in parts:
      offs.append(total)
      total += -(-n // 64) * 64  # 256-byte aligned parts
    plans.append((name, kwargs, plan))
    layout.append((parts, offs))
  block = t.empty(max(total, 1), dtype=t.int32, device=_native.device())
  base = _native.ptr(block)
  stats_base = _native.ptr(pending.stats_buffer)
  calls = []
  for i, ((name, kwargs, plan), (parts, offs)) in enumerate(zip(plans,
                                                                layout)):
    addr = [base + 4 * o for o in offs]
    out = _native.PreprocessOutput(
        addr[0], addr[1], addr[2], addr[3], stats_base + 4 * i * words,
        addr[4] if build_view else None, addr[5] if build_view else None)
    calls.append(_StackCall(plan.structs, plan.num_features, plan.opts, out,
                            plan.need))
  _preprocess_stacks(calls)
  for i, ((name, kwargs, plan), (parts, offs)) in enumerate(zip(plans,
                                                                layout)):
    rp, eid, sid, gains = (block[o:o + n] for o, n in zip(offs[:4],
                                                           parts[:4]))
    gains = gains.view(t.float32)
    view = None
    if build_view:
      view = (block[offs[4]:offs[4] + parts[4]],
              block[offs[5]:offs[5] + parts[5]].view(t.int64))
    stats_dev = pending.stats_buffer[i * words:(i + 1) * words]
    L, S, ns, off = plan.L, plan.S, plan.ns, plan.off
    feats = kwargs["feats"]
    if view is not None:
      sample_views[name] = view
    pending.append((name, stats_dev, L, S, ns, off, feats))
    jobs.append((name, kwargs))
    flat[name] = (rp, eid, sid, gains)
    if has_leading_dimension:
      rp, eid, sid, gains = (rp.reshape(L, -1), eid.reshape(L, -1),
                             sid.reshape(L, -1), gains.reshape(L, -1))
    rps[name], eids[name], sids[name], gns[name] = rp, eid, sid, gains
  if enable_minibatching:
    _minibatching_passes(pending, jobs, flat,
                         sample_views if sample_views is not None else {})
  else:
    # The stats go to the host behind the preprocessing, on its stream:
    # collect_stats then waits for this copy alone, not for whatever the
    # calling stream runs later.
    host = t.empty(pending.stats_buffer.numel(), dtype=t.int32,
                   pin_memory=True)
    host.copy_(pending.stats_buffer, non_blocking=True)
    ready = t.cuda.Event()
    ready.record()
    pending.host_stats, pending.host_stats_ready = host, ready
  return rps, eids, sids, gns, pending


def one_id_per_row(pending) -> dict:
  """Stack name -> whether every input row of the stack holds at most one
  id (then every activation row gets at most one CSR entry)."""
  out = {}
  for name, *_, feats in pending:
    ok = True
    for f in feats:
      ok = ok and f.one_id_per_row
    out[name] = ok
  return out


def collect_stats(pending) -> SparseDenseMatmulInputStats:
  """Waits for the enqueued preprocessing and returns its stats; raises as
  the reference does on bad ids or exceeded limits."""
  stats = SparseDenseMatmulInputStats()
  if not pending:
    return stats
  final = getattr(pending, "final_pass_stats", {})
  later = [final[p[0]] for p in pending if p[0] in final]
  # One wait for the first passes' stats and any later pass's counters.
  # The stacks' stats tensors are consecutive slices of stats_buffer.
  buffer = getattr(pending, "stats_buffer", None)
  early = getattr(pending, "host_stats", None)
  if early is not None and not later:
    pending.host_stats_ready.synchronize()
    host = early.numpy()
  else:
    host = _to_host(([buffer] if buffer is not None else
                     [p[1] for p in pending]) + [x[0] for x in later])
  pos = 0
  tail = sum(p[1].numel() for p in pending)
  for name, stats_dev, L, S, ns, off, _ in pending:
    stats_np = host[pos:pos + stats_dev.numel()]
    pos += stats_dev.numel()
    counters = stats_np[off:off + 2 * _NUM_COUNTERS].copy().view(np.int64)
    _raise_on_counters(name, counters)
    if name in final:
      later_dev, later_off = final[name]
      chunk = host[tail:tail + later_dev.numel()]
      tail += later_dev.numel()
      later_counters = chunk[later_off:later_off +
                             2 * _NUM_COUNTERS].copy().view(np.int64)
      _raise_on_counters(name, later_counters)
      # The stats stay the first pass's (input_preprocessing.cc:268-276);
      # the dropped ids are the final pass's.
      counters = counters.copy()
      counters[0] = later_counters[0]
      counters[3] = later_counters[3]
    stats.max_ids_per_partition[name] = stats_np[:L * ns].copy()
    stats.max_unique_ids_per_partition[name] = stats_np[L * ns:2 * L *
                                                        ns].copy()
    stats.required_buffer_sizes[name] = stats_np[2 * L * ns:2 * L * ns +
                                                 L * S].copy()
    stats.dropped_id_count[name] = int(counters[0])
    stats.num_entries[name] = int(counters[3])
  return stats


class RaggedIds:
  """Ids of one feature as flat values plus row splits (row r holds
  values[row_splits[r]:row_splits[r + 1]]); accepted wherever a feature is.
  `values` may be a numpy array or a CUDA tensor, `row_splits` is host
  int64 [batch + 1]."""

  def __init__(self, values, row_splits):
    self.values = values
    self.row_splits = row_splits


def sparse_coo_to_ragged(indices, values, dense_shape) -> RaggedIds:
  """A 2-D sparse tensor in COO form (tf.sparse.SparseTensor layout: indices
  [N, 2] row-major, values [N], dense_shape [batch, width]) as RaggedIds.

  Row splits as ConstructRowPointers builds them
  (lib/core/sparse_coo_input_batch.cc:30-66): row_splits[r] is the first
  entry whose row index is >= r, for r = 0..batch. The column index only
  orders the ids of a row. The reference DCHECKs row-major order; here a
  violation (decreasing row, non-increasing column within a row) or a row
  outside [0, batch) raises ValueError.
  """
  batch = int(np.asarray(
      dense_shape.cpu() if hasattr(dense_shape, "cpu") else dense_shape,
      np.int64).reshape(-1)[0])
  if hasattr(indices, "cpu"):  # a tensor: the checks read back once
    idx = indices.reshape(-1, 2)
    rows, cols = idx[:, 0], idx[:, 1]
    t = _native.torch()
    n = int(rows.shape[0])
    if n:
      same = rows[1:] == rows[:-1]
      bad = ((rows[1:] < rows[:-1]) | (same & (cols[1:] <= cols[:-1]))).any()
      flags = t.stack([bad, rows.min() < 0, rows.max() >= batch]).cpu()
      if bool(flags[0]):
        raise ValueError("sparse indices must be sorted in row-major order")
      if bool(flags[1]) or bool(flags[2]):
        raise ValueError(f"sparse row index outside [0, {batch})")
    splits = t.searchsorted(
        rows.contiguous(),
        t.arange(batch + 1, device=rows.device, dtype=rows.dtype))
    return RaggedIds(values.reshape(-1), splits.cpu().numpy().astype(np.int64))
  idx = np.asarray(indices, np.int64).reshape(-1, 2)
  rows, cols = idx[:, 0], idx[:, 1]
  if rows.size:
    d_row = np.diff(rows)
    if (d_row < 0).any() or ((d_row == 0) & (np.diff(cols) <= 0)).any():
      raise ValueError("sparse indices must be sorted in row-major order")
    if rows[0] < 0 or rows[-1] >= batch:
      raise ValueError(f"sparse row index outside [0, {batch})")
  splits = np.searchsorted(rows, np.arange(batch + 1), side="left")
  vals = values.reshape(-1) if hasattr(values, "data_ptr") else np.asarray(
      values, np.int32).reshape(-1)
  if vals.shape[0] != rows.shape[0]:
    raise ValueError("indices and values must have the same length")
  return RaggedIds(vals, splits.astype(np.int64))


def preprocess_sparse_dense_matmul_sparse_coo_input(
    indices,
    values,
    dense_shapes,
    feature_specs,
    local_device_count: int,
    global_device_count: int,
    *,
    num_sc_per_device: int,
    sharding_strategy=ShardingStrategy.MOD,
    has_leading_dimension: bool = False,
    allow_id_dropping: bool = False,
    batch_number: int = 0,
    enable_minibatching: bool = False,
    all_reduce_interface=None,
):
  """PySparseCooPreprocessSparseDenseMatmulInput
  (pybind_input_preprocessing.cc:250-276): one sparse COO tensor per feature,
  unity weights; same outputs as preprocess_sparse_dense_matmul_input."""
  indices, values, dense_shapes = list(indices), list(values), list(
      dense_shapes)
  if not len(indices) == len(values) == len(dense_shapes):
    raise ValueError("indices, values and dense_shapes must have equal length")
  features = [sparse_coo_to_ragged(i, v, d)
              for i, v, d in zip(indices, values, dense_shapes)]
  return preprocess_sparse_dense_matmul_input(
      features, None, feature_specs, local_device_count, global_device_count,
      num_sc_per_device=num_sc_per_device,
      sharding_strategy=sharding_strategy,
      has_leading_dimension=has_leading_dimension,
      allow_id_dropping=allow_id_dropping, batch_number=batch_number,
      enable_minibatching=enable_minibatching,
      all_reduce_interface=all_reduce_interface)
