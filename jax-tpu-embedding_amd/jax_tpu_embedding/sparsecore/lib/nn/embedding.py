"""Embedding API for the MI355X SparseCore path (reference: lib/nn/embedding.py).

Same entry points, arguments and results as the reference module:
  preprocess_sparse_dense_matmul_input   (:608-705)  -> GPU preprocessing
  tpu_sparse_dense_matmul                (:1047-1184) -> forward lookup
  tpu_sparse_dense_matmul_grad           (:1297-1529) -> backward + optimizer
  stack_embedding_gradients / unstack_embedding_activations (:903-1294)
  prepare_feature_specs_for_training, auto_stack_tables, size helpers,
  init_embedding_variables, update_preprocessing_parameters.
Arrays are torch tensors on the GPU (numpy inputs are copied there). Tables
and slots are updated in place by the gradient step, which returns them.
"""

from __future__ import annotations

import collections
import dataclasses
import functools
import warnings
from typing import Mapping, NamedTuple

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore import _tree
from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_activation_unstack
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_gradient_stack
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils as prim_utils
from jax_tpu_embedding.sparsecore.lib.nn import custom_optimizer_lowering
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from jax_tpu_embedding.sparsecore.lib.nn import table_stacking
from jax_tpu_embedding.sparsecore.utils import utils

LimitsCallable = table_stacking.LimitsCallable
get_default_limits = table_stacking.get_default_limits


def _assert_same_structure(a, b, a_name="a", b_name="b"):
  if _tree.leaf_paths(a) != _tree.leaf_paths(b):
    raise ValueError(f"Pytree structures of {a_name} and {b_name} do not "
                     "match.")


class EmbeddingVariables(NamedTuple):
  table: object
  slot: tuple


class SparseDenseMatmulInput(NamedTuple):
  """The CSR-wrapped COO buffers per stacked table."""

  lhs_row_pointers: Mapping
  lhs_embedding_ids: Mapping
  lhs_sample_ids: Mapping
  lhs_gains: Mapping


@dataclasses.dataclass
class SparseDenseMatmulInputStats:
  """Preprocessing stats per stacked table (embedding.py:97-188)."""

  # The suffixes name each field's entries in FDO stats files
  # (lib/fdo/file_fdo_client.py: "<table><suffix>").
  max_ids_per_partition: dict = dataclasses.field(
      default_factory=dict, metadata={"suffix": "_max_ids"})
  max_unique_ids_per_partition: dict = dataclasses.field(
      default_factory=dict, metadata={"suffix": "_max_unique_ids"})
  required_buffer_size_per_sc: dict = dataclasses.field(
      default_factory=dict, metadata={"suffix": "_required_buffer_size"})
  id_drop_counters: dict = dataclasses.field(
      default_factory=dict, metadata={"suffix": "_id_drop_counters"})

  @classmethod
  def from_cc(cls, stats) -> "SparseDenseMatmulInputStats":
    return cls(
        max_ids_per_partition=stats.max_ids_per_partition,
        max_unique_ids_per_partition=stats.max_unique_ids_per_partition,
        required_buffer_size_per_sc=stats.required_buffer_sizes,
        id_drop_counters=stats.dropped_id_count,
    )

  def get_required_buffer_size_per_device(self, table_name: str,
                                          num_sc_per_device: int | None = None):
    if table_name not in self.required_buffer_size_per_sc:
      return None
    val = self.required_buffer_size_per_sc[table_name]
    num_sc = num_sc_per_device or np.size(val)
    return int(np.max(val) * num_sc)

  def set_required_buffer_size_per_device(self, table_name: str,
                                          required_buffer_size_per_device: int,
                                          num_sc_per_device: int | None = None):
    val = self.required_buffer_size_per_sc.get(table_name)
    num_sc = num_sc_per_device or (np.size(val) if val is not None else 0)
    if not num_sc:
      raise ValueError(
          "num_sc_per_device must be provided if the table is not present.")
    self.required_buffer_size_per_sc[table_name] = np.full(
        num_sc, required_buffer_size_per_device / num_sc)


@dataclasses.dataclass
class PreprocessedInput:
  """Result of preprocessing: the CSR buffers and the minibatch count.

  Two optional fields have no reference counterpart; the GPU preprocessing
  fills them and the lookup uses them when present:
    lookup_views: stack name -> _native.LookupView, the CSR entries grouped
      by activation row (spares the forward pass its grouping sort);
    csr_sorted_by_row: whether the CSR entries are ascending by (partition,
      embedding id) in every segment (with minibatching: every row's
      entries contiguous), which lets the backward pass read the CSR in
      place; None (the default) takes that order from the reference's
      format, which always has it;
    csr_num_entries: stack name -> number of CSR entries (lets the lookup
      pick the kernel variant for one-hot or multi-hot batches).
  A PreprocessedInput built from other CSR buffers leaves them unset.
  """

  sparse_dense_matmul_input: SparseDenseMatmulInput
  num_minibatches: object = dataclasses.field(
      default_factory=lambda: np.array(1))
  lookup_views: dict | None = None
  csr_sorted_by_row: bool | None = None
  csr_num_entries: dict | None = None

  @property
  def lhs_row_pointers(self):
    return self.sparse_dense_matmul_input.lhs_row_pointers

  @property
  def lhs_embedding_ids(self):
    return self.sparse_dense_matmul_input.lhs_embedding_ids

  @property
  def lhs_sample_ids(self):
    return self.sparse_dense_matmul_input.lhs_sample_ids

  @property
  def lhs_gains(self):
    return self.sparse_dense_matmul_input.lhs_gains

  def __iter__(self):
    warnings.warn(
        "Please use attributed lookup on sparse_dense_matmul_input attribute.",
        DeprecationWarning)
    return iter(self.sparse_dense_matmul_input)


def _verify_feature_specs(feature_specs) -> None:
  seen = set()
  for fs in _tree.tree_leaves(feature_specs):
    if fs.name in seen:
      raise ValueError(f"Feature spec {fs.name} is already defined.")
    seen.add(fs.name)


def _get_num_sc_per_device(num_sc_per_device: int | None) -> int:
  if num_sc_per_device is None:
    return utils.num_sparsecores_per_device()
  if num_sc_per_device not in utils.NUM_SC_PER_DEVICE_MAP.values():
    raise ValueError(f"Invalid num_sc_per_device: {num_sc_per_device}")
  return num_sc_per_device


def get_table_specs(feature_specs):
  _verify_feature_specs(feature_specs)
  out = {}
  for fs in _tree.tree_leaves(feature_specs):
    out[fs.table_spec.name] = fs.table_spec
  return out


def get_stacked_table_specs(feature_specs):
  _verify_feature_specs(feature_specs)
  leaves = _tree.tree_leaves(feature_specs)
  if any(not fs.table_spec.is_stacked() for fs in leaves):
    raise ValueError(
        "embedding.prepare_feature_specs_for_training was not called")
  return {fs.table_spec.stacked_table_spec.stack_name:
          fs.table_spec.stacked_table_spec for fs in leaves}


def prepare_feature_specs_for_training(feature_specs, global_device_count: int,
                                       num_sc_per_device: int | None = None):
  """Gives every unstacked table a stack of its own and stacks the features
  that share a table (embedding.py:342-453)."""
  num_sc_per_device = _get_num_sc_per_device(num_sc_per_device)
  leaves = _tree.tree_leaves(feature_specs)
  not_stacked = [f for f in leaves if not f.table_spec.is_stacked()]
  by_table = collections.defaultdict(list)
  for f in not_stacked:
    by_table[f.table_spec.name].append(f)
  row_offsets = {}
  for features in by_table.values():
    offset = 0
    for f in sorted(features, key=lambda f: f.name):
      row_offsets[f.name] = offset
      offset += int(np.prod(f.output_shape[:-1]))
  ns = num_sc_per_device * global_device_count
  for f in leaves:
    if f not in not_stacked:
      continue
    t = f.table_spec
    s = t._setting_in_stack  # pylint: disable=protected-access
    if s is not None and s.stack_name != t.name:
      raise ValueError(
          f"Invalid stacking. Table {t.name} does not have StackedTableSpec "
          f"populated, but feature.table_spec.setting_in_stack.stack_name "
          f"({s.stack_name}) is not {t.name}.")
    dims, vocabs = table_stacking.round_up_dim_and_vocab_size({t.name: t}, ns)
    total = sum(int(np.prod(g.output_shape[:-1])) for g in by_table[t.name])
    t.setting_in_stack = embedding_spec.TableSettingInStack(
        stack_name=t.name, padded_embedding_dim=dims[t.name],
        padded_vocab_size=vocabs[t.name], row_offset_in_shard=0,
        shard_rotation=0)
    t.stacked_table_spec = embedding_spec.StackedTableSpec(
        stack_name=t.name, stack_vocab_size=vocabs[t.name],
        stack_embedding_dim=dims[t.name], optimizer=t.optimizer,
        combiner=t.combiner, total_sample_count=total,
        max_ids_per_partition=t.max_ids_per_partition,
        max_unique_ids_per_partition=t.max_unique_ids_per_partition,
        suggested_coo_buffer_size_per_device=(
            t.suggested_coo_buffer_size_per_device),
        quantization_config=t.quantization_config)
    f.id_transformation = embedding_spec.FeatureIdTransformation(
        row_offset=row_offsets.get(f.name, 0), col_offset=0, col_shift=0)


def auto_stack_tables(feature_specs, global_device_count: int,
                      num_sc_per_device: int | None = None,
                      stack_to_max_ids_per_partition=get_default_limits,
                      stack_to_max_unique_ids_per_partition=get_default_limits,
                      use_short_stack_names: bool = True, *,
                      activation_mem_bytes_limit: int | None = None) -> None:
  num_sc_per_device = _get_num_sc_per_device(num_sc_per_device)
  table_stacking.auto_stack_tables(
      feature_specs, global_device_count=global_device_count,
      num_sc_per_device=num_sc_per_device,
      stack_to_max_ids_per_partition=stack_to_max_ids_per_partition,
      stack_to_max_unique_ids_per_partition=(
          stack_to_max_unique_ids_per_partition),
      use_short_stack_names=use_short_stack_names,
      activation_mem_bytes_limit=activation_mem_bytes_limit)


def compute_row_pointers_size_per_device(*, global_device_count: int,
                                         num_sc_per_device: int | None = None,
                                         enable_minibatching: bool = False):
  return pybind_input_preprocessing.compute_row_pointers_size_per_device(
      global_device_count=global_device_count,
      num_sc_per_device=_get_num_sc_per_device(num_sc_per_device),
      enable_minibatching=enable_minibatching)


def compute_theoretical_max_coo_buffer_size(max_ids_per_partition: int,
                                            global_device_count: int,
                                            num_sc_per_device: int | None = None,
                                            enable_minibatching: bool = False):
  return pybind_input_preprocessing.compute_theoretical_max_coo_buffer_size(
      max_ids_per_partition=max_ids_per_partition,
      global_device_count=global_device_count,
      num_sc_per_device=_get_num_sc_per_device(num_sc_per_device),
      enable_minibatching=enable_minibatching)


def compute_coo_buffer_size_per_device(feature_specs, global_device_count: int,
                                       num_sc_per_device: int | None = None,
                                       enable_minibatching: bool = False):
  return pybind_input_preprocessing.compute_coo_buffer_size_per_device(
      feature_specs=_tree.tree_leaves(feature_specs),
      global_device_count=global_device_count,
      num_sc_per_device=_get_num_sc_per_device(num_sc_per_device),
      enable_minibatching=enable_minibatching)


# Shape and dtype of an array that is not materialised (the two fields of
# jax.ShapeDtypeStruct).
ShapeDtypeStruct = prim_utils.ShapedArray


def eval_preprocess_sparse_dense_matmul_input_shape(
    feature_specs, local_device_count: int, global_device_count: int, *,
    num_sc_per_device: int | None = None, has_leading_dimension: bool = False,
    enable_minibatching: bool = False) -> PreprocessedInput:
  """Shapes and dtypes of preprocess_sparse_dense_matmul_input's outputs
  from the specs alone, without input tensors or a device
  (embedding.py:822-900): per stacked table the row pointers, embedding ids,
  sample ids and gains as flat `(local_device_count * size,)` arrays (the
  COO size from compute_coo_buffer_size_per_device, the row-pointer size
  from compute_row_pointers_size_per_device, 64 times larger with
  minibatching), and the minibatch counts as `(local_device_count,)` int32,
  `(local_device_count, 1)` with `has_leading_dimension`. The leaves are
  ShapeDtypeStruct records in a PreprocessedInput."""
  coo = compute_coo_buffer_size_per_device(
      feature_specs, global_device_count, num_sc_per_device=num_sc_per_device,
      enable_minibatching=enable_minibatching)
  rp_size = compute_row_pointers_size_per_device(
      global_device_count=global_device_count,
      num_sc_per_device=num_sc_per_device,
      enable_minibatching=enable_minibatching)

  def flat(size, dtype):
    return ShapeDtypeStruct((local_device_count * size,), dtype)

  nmb = ShapeDtypeStruct(
      (local_device_count, 1) if has_leading_dimension else
      (local_device_count,), np.int32)
  return PreprocessedInput(
      sparse_dense_matmul_input=SparseDenseMatmulInput(
          lhs_row_pointers={k: flat(rp_size, np.int32) for k in coo},
          lhs_embedding_ids={k: flat(n, np.int32) for k, n in coo.items()},
          lhs_sample_ids={k: flat(n, np.int32) for k, n in coo.items()},
          lhs_gains={k: flat(n, np.float32) for k, n in coo.items()}),
      num_minibatches=nmb)


def sharding_strategy_to_enum(sharding_strategy: str):
  if sharding_strategy.upper() == "MOD":
    return pybind_input_preprocessing.ShardingStrategy.MOD
  raise ValueError(f"Unsupported sharding strategy: {sharding_strategy}. "
                   "Only MOD is supported.")


def preprocess_sparse_dense_matmul_input(
    features, features_weights, feature_specs, local_device_count: int,
    global_device_count: int, *, num_sc_per_device: int | None = None,
    sharding_strategy: str = "MOD", has_leading_dimension: bool = False,
    allow_id_dropping: bool = False, batch_number: int = 0,
    enable_minibatching: bool = False, all_reduce_interface=None):
  """Preprocesses the input batch on the GPU (embedding.py:608-705).

  Returns (PreprocessedInput, SparseDenseMatmulInputStats); the CSR buffers
  are torch CUDA tensors.
  """
  preprocessed, stats = enqueue_preprocess_sparse_dense_matmul_input(
      features, features_weights, feature_specs, local_device_count,
      global_device_count, num_sc_per_device=num_sc_per_device,
      sharding_strategy=sharding_strategy,
      has_leading_dimension=has_leading_dimension,
      allow_id_dropping=allow_id_dropping, batch_number=batch_number,
      enable_minibatching=enable_minibatching,
      all_reduce_interface=all_reduce_interface)
  return preprocessed, stats.result()


class PreprocessStats:
  """The stats of a preprocessing call still running on the device
  (enqueue_preprocess_sparse_dense_matmul_input). result() waits for them
  (for the copy enqueued behind the call on its stream, not for later work
  on that stream), raises as preprocess_sparse_dense_matmul_input does on
  ids outside a table or over the limits, records the entry counts in the
  PreprocessedInput (the lookup picks kernel variants by them; until then
  it sizes by the buffers) and returns SparseDenseMatmulInputStats."""

  def __init__(self, pending, preprocessed, enable_minibatching):
    self._pending = pending
    self._preprocessed = preprocessed
    self._minibatching = enable_minibatching
    self._stats = None

  def result(self) -> SparseDenseMatmulInputStats:
    if self._stats is not None:
      return self._stats
    stats = pybind_input_preprocessing.collect_stats(self._pending)
    pre = self._preprocessed
    if pre.lookup_views is not None:
      counts = dict(stats.num_entries)
      pre.csr_num_entries = counts
      for name, view in pre.lookup_views.items():
        view.num_entries = counts.get(name, 0)
        if self._minibatching and view.num_entries:
          # The view has room for a buffer sized for 64 minibatches; past
          # the entries it holds only unused keys.
          used = -(-view.num_entries // 256) * 256
          if used < view.keys.numel():
            view.keys, view.entries = view.keys[:used], view.entries[:used]
    self._stats = SparseDenseMatmulInputStats.from_cc(stats)
    self._pending = None
    return self._stats


def enqueue_preprocess_sparse_dense_matmul_input(
    features, features_weights, feature_specs, local_device_count: int,
    global_device_count: int, *, num_sc_per_device: int | None = None,
    sharding_strategy: str = "MOD", has_leading_dimension: bool = False,
    allow_id_dropping: bool = False, batch_number: int = 0,
    enable_minibatching: bool = False, all_reduce_interface=None):
  """preprocess_sparse_dense_matmul_input without the wait: enqueues the
  preprocessing on the current stream and returns (PreprocessedInput,
  PreprocessStats) at once (no counterpart in the reference, whose
  preprocessing runs on the host). Work enqueued later on the stream may use
  the PreprocessedInput; a training loop can preprocess batch k + 1 on a
  second stream during step k and call result() once step k + 1 is
  enqueued. Arguments are checked before anything is enqueued; ids outside
  a table and exceeded limits are raised by result(). Minibatching decides
  between its passes on the host, so with enable_minibatching this waits
  for the first pass."""
  num_sc_per_device = _get_num_sc_per_device(num_sc_per_device)
  _assert_same_structure(features, feature_specs, "features", "feature_specs")
  if features_weights is not None:
    _assert_same_structure(features_weights, feature_specs,
                           "features_weights", "feature_specs")
  if (enable_minibatching and all_reduce_interface is None and
      local_device_count < global_device_count):
    raise ValueError("all_reduce_interface must be provided when minibatching "
                     "is enabled for multi-host.")
  del batch_number
  feats, weights, specs = pybind_input_preprocessing.check_arguments(
      _tree.tree_leaves(features),
      (_tree.tree_leaves(features_weights)
       if features_weights is not None else None),
      _tree.tree_leaves(feature_specs),
      sharding_strategy_to_enum(sharding_strategy), enable_minibatching,
      local_device_count=local_device_count,
      global_device_count=global_device_count,
      num_sc_per_device=num_sc_per_device)
  # Everything is enqueued (CSR build, then the lookup views) before the one
  # wait for the stats.
  built = {}
  *csr, pending = pybind_input_preprocessing.enqueue_preprocessing(
      feats, weights, specs, local_device_count, global_device_count,
      num_sc_per_device=num_sc_per_device,
      has_leading_dimension=has_leading_dimension,
      allow_id_dropping=allow_id_dropping, sample_views=built,
      enable_minibatching=enable_minibatching)
  views = None
  if local_device_count == 1:
    # One device: the preprocessing wrote each stack's sample view along with
    # its CSR; otherwise (several global devices) it is built from the CSR.
    stacked = get_stacked_table_specs(feature_specs)
    one_per_row = pybind_input_preprocessing.one_id_per_row(pending)
    views = {
        name: _native.LookupView(
            keys, entries, stacked[name].total_sample_count,
            stacked[name].stack_vocab_size,
            one_entry_per_key=one_per_row.get(name, False))
        for name, (keys, entries) in built.items()}
    missing = [n for n in stacked if n not in views]
    if missing:
      views.update(_build_lookup_views(
          csr, feature_specs, global_device_count, num_sc_per_device,
          one_per_row, only=missing,
          num_minibatches=(pending.num_minibatches if enable_minibatching
                           else 0)))
  minibatches = np.full(local_device_count, pending.num_minibatches,
                        dtype=np.int32)
  if has_leading_dimension:
    minibatches = minibatches.reshape(local_device_count, 1)
  preprocessed = PreprocessedInput(
      SparseDenseMatmulInput(*csr), minibatches, lookup_views=views,
      csr_sorted_by_row=(None if local_device_count == 1 else False),
      csr_num_entries=None)
  return preprocessed, PreprocessStats(pending, preprocessed,
                                       enable_minibatching)


def preprocess_sparse_dense_matmul_input_from_sparse_tensor(
    indices, values, dense_shapes, feature_specs, local_device_count: int,
    global_device_count: int, *, num_sc_per_device: int | None = None,
    sharding_strategy: str = "MOD", has_leading_dimension: bool = False,
    allow_id_dropping: bool = False, batch_number: int = 0,
    enable_minibatching: bool = False, all_reduce_interface=None):
  """Preprocesses sparse COO features on the GPU (embedding.py:708-806).

  `indices` ([N, 2] row-major), `values` ([N] ids) and `dense_shapes`
  ([batch, width]) share the structure of `feature_specs`; weights are 1.
  Each feature becomes flat ids plus row splits
  (pybind_input_preprocessing.sparse_coo_to_ragged) and goes through the same
  preprocessing as preprocess_sparse_dense_matmul_input.
  """
  _assert_same_structure(indices, feature_specs, "indices", "feature_specs")
  _assert_same_structure(values, feature_specs, "values", "feature_specs")
  _assert_same_structure(dense_shapes, feature_specs, "dense_shapes",
                         "feature_specs")
  specs = _tree.tree_leaves(feature_specs)
  features = [
      pybind_input_preprocessing.sparse_coo_to_ragged(i, v, d)
      for i, v, d in zip(_tree.tree_leaves(indices), _tree.tree_leaves(values),
                         _tree.tree_leaves(dense_shapes))
  ]
  return preprocess_sparse_dense_matmul_input(
      features, None, specs, local_device_count, global_device_count,
      num_sc_per_device=num_sc_per_device,
      sharding_strategy=sharding_strategy,
      has_leading_dimension=has_leading_dimension,
      allow_id_dropping=allow_id_dropping, batch_number=batch_number,
      enable_minibatching=enable_minibatching,
      all_reduce_interface=all_reduce_interface)


def _build_lookup_views(csr, feature_specs, global_device_count: int,
                        num_sc_per_device: int, one_per_row: dict,
                        only=None, num_minibatches: int = 0):
  """Sample views of one device's CSR buffers, one per stacked table (those
  named in `only`, when given), for a table shard of
  stack_vocab_size / global_device_count rows."""
  rp, eid, sid, gains = csr
  views = {}
  for name, spec in get_stacked_table_specs(feature_specs).items():
    if only is not None and name not in only:
      continue
    batch = spec.total_sample_count // global_device_count
    rows = spec.stack_vocab_size // global_device_count
    _, c = _device.csr_operands(rp[name], eid[name], sid[name], gains[name],
                                num_sc_per_device,
                                num_sc_per_device * global_device_count,
                                one_entry_per_row=one_per_row.get(name, False),
                                num_minibatches=num_minibatches)
    views[name] = _native.build_sample_view(c, batch, rows)
  return views


# ---------------------------------------------------------------------------
# Activation unstacking / gradient stacking (embedding.py:903-1044,
# :1200-1294): layout changes between the stacked [B_stack, D] buffer and
# per-feature [b_f, d_f] arrays.
# ---------------------------------------------------------------------------


def _get_activation_for_feature(feature, activations, global_device_count,
                                num_feature_slices_per_device):
  if feature.output_shape[-1] > feature.table_spec.embedding_dim:
    raise ValueError(
        f"Feature {feature.name} has output shape {feature.output_shape} and "
        f"embedding dim {feature.table_spec.embedding_dim}. The embedding dim "
        "in output shape cannot be more than the (original, unpadded) "
        "embedding dim in the FeatureSpec.")
  act = activations[feature.table_spec.stacked_table_spec.stack_name]
  f = num_feature_slices_per_device
  if act.shape[0] % f:
    raise ValueError(
        "The input batch size must be divisible by the number of feature "
        f"slices per device. Got input shape {tuple(act.shape)} and {f} "
        f"feature slices per device for feature {feature.name}.")
  off = feature.id_transformation.row_offset // (global_device_count * f)
  b1 = feature.output_shape[0] // (global_device_count * f)
  if f == 1:
    # One slice per device: a row range (and leading columns) of the
    # stacked activations.
    sl = act.narrow(0, off, b1)
    if act.dim() > 1 and feature.output_shape[-1] < act.shape[-1]:
      sl = sl.narrow(-1, 0, feature.output_shape[-1])
    return sl
  per = act.reshape(f, act.shape[0] // f, *act.shape[1:])
  sl = per[:, off:off + b1]
  if act.dim() > 1:
    sl = sl[..., :feature.output_shape[-1]]
  return sl.reshape(f * b1, *sl.shape[2:])


def _activation_blocks(stack_spec, features, global_device_count: int,
                       num_sc_per_device: int, dev):
  """Per-feature outputs of one stacked table and the RowBlocks that let the
  forward kernel write them directly (the layout _get_activation_for_feature
  slices out of the stacked activations). None when plain views of the
  stacked activations already are the outputs (one SparseCore, every feature
  at the full stacked dim) or the stack needs more blocks than the kernels
  take."""
  t = _native.torch()
  f = num_sc_per_device
  rows = stack_spec.total_sample_count // global_device_count
  dim = stack_spec.stack_embedding_dim
  if len(features) * f > _native.MAX_ROW_BLOCKS or rows % f:
    return None
  if f == 1 and all(fs.output_shape[-1] == dim for fs in features):
    return None
  widths = []
  for fs in features:
    if fs.output_shape[-1] > fs.table_spec.embedding_dim:
      raise ValueError(
          f"Feature {fs.name} has output shape {fs.output_shape} and "
          f"embedding dim {fs.table_spec.embedding_dim}. The embedding dim "
          "in output shape cannot be more than the (original, unpadded) "
          "embedding dim in the FeatureSpec.")
    widths.append(fs.output_shape[-1])
  # One allocation per stack; each feature's output is a contiguous slice.
  sizes = [f * (fs.output_shape[0] // (global_device_count * f)) * w
           for fs, w in zip(features, widths)]
  flat = t.empty(sum(sizes), dtype=t.float32, device=dev)
  outs, blocks, start = {}, [], 0
  for fs, width, size in zip(features, widths, sizes):
    off = fs.id_transformation.row_offset // (global_device_count * f)
    b1 = fs.output_shape[0] // (global_device_count * f)
    out = flat[start:start + size].view(f * b1, width)
    start += size
    outs[fs.name] = out
    for s in range(f):
      blocks.append((s * (rows // f) + off, out[s * b1:(s + 1) * b1], width))
  blocks.sort(key=lambda b: b[0])
  return outs, _device.RowBlocks(rows, dim, blocks)


def _gradient_blocks(stack_spec, items, num_sc_per_device: int,
                     num_entries=None):
  """RowBlocks over the per-feature gradients of one stacked table, in the
  layout stack_embedding_gradients builds; None when the stack needs more
  blocks than the kernels take or is multi-hot (`num_entries`, the CSR's
  entries, above twice its rows)."""
  f = num_sc_per_device
  if len(items) * f > _native.MAX_ROW_BLOCKS:
    return None
  if num_entries is not None and num_entries > 2 * sum(
      int(fs.output_shape[0]) for fs, _ in items):
    # Multi-hot: every gradient row is gathered many times; one stacking
    # copy costs less than resolving the row blocks per gather.
    return None
  t = _native.torch()
  dev = _native.device()
  grads = []
  for fs, g in items:
    g = _native.as_device_tensor(g, t.float32, dev).reshape(
        -1, fs.table_spec.embedding_dim)
    if g.shape[0] % f:
      raise ValueError(
          "The input batch size must be divisible by the number of feature "
          f"slices per device. Got input shape {tuple(g.shape)} and "
          f"{f} feature slices per device for feature {fs.name}.")
    grads.append((fs, g))
  rows = sum(g.shape[0] for _, g in grads)
  per_sc = rows // f
  blocks, cum = [], 0
  for fs, g in grads:
    b1 = g.shape[0] // f
    if f == 1:
      blocks.append((cum, g, fs.table_spec.embedding_dim))
    else:
      for s in range(f):
        blocks.append((s * per_sc + cum, g[s * b1:(s + 1) * b1],
                       fs.table_spec.embedding_dim))
    cum += b1
  blocks.sort(key=lambda b: b[0])
  return _device.RowBlocks(rows, stack_spec.stack_embedding_dim, blocks)


def _unstack_activations_with_primitive(activations, feature_specs,
                                        global_device_count: int,
                                        num_sc_per_device: int):
  """Unstacking through tpu_sparse_dense_matmul_activation_unstack_primitive
  (embedding.py:971-1028): one call per stacked table over its features in
  row-offset order, each feature at its table's embedding dim."""
  flat, treedef = _tree.tree_flatten(feature_specs)
  out = [None] * len(flat)
  by_stack = collections.defaultdict(list)
  for i, fs in enumerate(flat):
    if any(d is None for d in fs.output_shape):
      raise ValueError(
          f"Feature {fs.name} has dynamic output shape {fs.output_shape}, "
          "which is not supported.")
    by_stack[fs.table_spec.stacked_table_spec.stack_name].append((i, fs))
  for name, items in by_stack.items():
    items.sort(key=lambda x: x[1].id_transformation.row_offset)
    batches = tuple(int(np.prod(fs.output_shape[:-1])) // global_device_count
                    for _, fs in items)
    dims = tuple(fs.table_spec.embedding_dim for _, fs in items)
    acts = (sparse_dense_matmul_activation_unstack
            .tpu_sparse_dense_matmul_activation_unstack_primitive.bind(
                activations[name], per_feature_batch_sizes=batches,
                per_feature_dims=dims, num_sc_per_device=num_sc_per_device))
    for (i, _), a in zip(items, acts):
      out[i] = a
  return _tree.tree_unflatten(treedef, out)


def unstack_embedding_activations(activations, feature_specs,
                                  global_device_count: int,
                                  num_sc_per_device: int,
                                  use_activation_unstack_primitive=False):
  """Per-feature activations from the stacked ones (embedding.py:1031-1044):
  views of the stacked activations, or with
  `use_activation_unstack_primitive` new tensors copied out by the
  unstacking primitive."""
  if use_activation_unstack_primitive:
    return _unstack_activations_with_primitive(
        activations, feature_specs, global_device_count, num_sc_per_device)
  return _tree.tree_map(
      lambda fs: _get_activation_for_feature(fs, activations,
                                             global_device_count,
                                             num_sc_per_device),
      feature_specs)


def tpu_sparse_dense_matmul(preprocessed_inputs, embedding_variables,
                            feature_specs, *, global_device_count: int,
                            sharding_strategy: str = "MOD",
                            num_sc_per_device: int | None = None,
                            enable_minibatching: bool = False,
                            perform_unstacking: bool = True,
                            use_activation_unstack_primitive: bool = False):
  """Forward lookup for every stacked table (embedding.py:1047-1184)."""
  if isinstance(preprocessed_inputs, SparseDenseMatmulInput):
    warnings.warn("SparseDenseMatmulInput is deprecated. Please use "
                  "PreprocessedInput instead.", DeprecationWarning)
    preprocessed_inputs = PreprocessedInput(preprocessed_inputs)
  rp, eid, sid, gains = preprocessed_inputs.sparse_dense_matmul_input
  num_sc_per_device = _get_num_sc_per_device(num_sc_per_device)
  assert rp.keys() == embedding_variables.keys()
  stacked = get_stacked_table_specs(feature_specs)
  assert rp.keys() == stacked.keys()
  strategy = int(sharding_strategy_to_enum(sharding_strategy))
  nmb = _resolve_scalar_minibatches(preprocessed_inputs.num_minibatches)
  views = getattr(preprocessed_inputs, "lookup_views", None) or {}
  counts = getattr(preprocessed_inputs, "csr_num_entries", None) or {}
  leaves = _tree.tree_leaves(feature_specs)
  by_stack = collections.defaultdict(list)
  for fs in leaves:
    by_stack[fs.table_spec.stacked_table_spec.stack_name].append(fs)
  per_feature = {}

  def lookup(name):
    spec = stacked[name]
    ev = embedding_variables[name]
    table = ev.table if isinstance(ev, EmbeddingVariables) else ev[0]
    fused = None
    if (perform_unstacking and not use_activation_unstack_primitive and
        len(getattr(table, "shape", ())) == 2):
      # Unstacking fused into the kernel: activation rows go straight to
      # the per-feature outputs.
      fused = _activation_blocks(spec, by_stack[name], global_device_count,
                                 num_sc_per_device, _native.device())
    act = (sparse_dense_matmul_csr.tpu_sparse_dense_matmul_csr_primitive
           .bind(rp[name], eid[name], sid[name], gains[name], nmb, table,
                 device_batch_size=(spec.total_sample_count //
                                    global_device_count),
                 max_ids_per_partition=spec.max_ids_per_partition,
                 max_unique_ids_per_partition=(
                     spec.max_unique_ids_per_partition),
                 sharding_strategy=strategy,
                 quantization_config=(
                     spec.quantization_config.as_tuple()
                     if spec.quantization_config else None),
                 enable_minibatching=enable_minibatching,
                 num_sc_per_device=num_sc_per_device,
                 global_device_count=global_device_count,
                 lookup_view=views.get(name),
                 csr_num_entries=counts.get(name),
                 activation_blocks=fused[1] if fused else None))
    return act, fused

  # Independent stacks of different widths run concurrently (one side
  # stream per width); a quantized stack is refused inside its call.
  results = _native.run_per_stack(
      stacked.keys(), lookup, lambda n: stacked[n].stack_embedding_dim)
  acts = {}
  for name in stacked:
    acts[name], fused = results[name]
    if fused:
      per_feature.update(fused[0])
  if not perform_unstacking:
    return acts
  rest = [fs for fs in leaves if fs.name not in per_feature]
  if rest:
    stacked_acts = {k: v for k, v in acts.items()
                    if not isinstance(v, _device.RowBlocks)}
    unstacked = unstack_embedding_activations(
        stacked_acts, rest, global_device_count, num_sc_per_device,
        use_activation_unstack_primitive)
    per_feature.update({fs.name: a for fs, a in zip(rest, unstacked)})
  return _tree.tree_map(lambda fs: per_feature[fs.name], feature_specs)


def _resolve_scalar_minibatches(val):
  if isinstance(val, np.ndarray) and val.ndim == 1:
    return val[0].astype(np.int32)
  return val


def _prepare_gradient_for_stacking(gradient, feature, num_sc_per_device):
  t = _native.torch()
  g = gradient
  if not isinstance(g, t.Tensor):
    g = _native.as_device_tensor(g, t.float32)
  g = g.reshape(-1, feature.table_spec.embedding_dim)
  extra = (feature.table_spec.setting_in_stack.padded_embedding_dim -
           feature.table_spec.embedding_dim)
  if extra:
    g = t.nn.functional.pad(g, (0, extra))
  if g.shape[0] % num_sc_per_device:
    raise ValueError(
        "The input batch size must be divisible by the number of feature "
        f"slices per device. Got input shape {tuple(g.shape)} and "
        f"{num_sc_per_device} feature slices per device for feature "
        f"{feature.name}.")
  return g


def stack_embedding_gradients(activation_gradients, feature_specs,
                              num_sc_per_device: int,
                              global_device_count: int | None = None,
                              use_gradient_stacking_primitive: bool = False):
  """Per-feature gradients -> one [B_stack, D] gradient per stack
  (embedding.py:1220-1294): a concatenation per SparseCore slice, or with
  `use_gradient_stacking_primitive` one call of the stacking primitive per
  stacked table."""
  t = _native.torch()
  if use_gradient_stacking_primitive and global_device_count is None:
    raise ValueError("global_device_count must be provided when "
                     "use_gradient_stacking_primitive is True")
  by_stack = collections.defaultdict(list)
  for g, fs in zip(_tree.tree_leaves(activation_gradients),
                   _tree.tree_leaves(feature_specs)):
    if fs._id_transformation is None:  # pylint: disable=protected-access
      raise ValueError("FeatureIdTransformation cannot be None here. It is "
                       f"None for {fs.name}")
    by_stack[fs.table_spec.stacked_table_spec.stack_name].append((fs, g))
  out = {}
  f = num_sc_per_device
  for name, items in by_stack.items():
    items.sort(key=lambda x: x[0].id_transformation.row_offset)
    grads = [_prepare_gradient_for_stacking(g, fs, f) for fs, g in items]
    if use_gradient_stacking_primitive:
      spec = items[0][0].table_spec.stacked_table_spec
      out[name] = (sparse_dense_matmul_gradient_stack
                   .tpu_sparse_dense_matmul_gradient_stack_primitive.bind(
                       *grads,
                       stacked_batch_size=(spec.total_sample_count //
                                           global_device_count),
                       stacked_feature_dim=spec.stack_embedding_dim,
                       num_sc_per_device=f))
      continue
    parts = []
    for g in grads:
      parts.append(g.reshape(f, g.shape[0] // f, g.shape[1]))
    cat = t.cat(parts, dim=1)
    out[name] = cat.reshape(-1, cat.shape[-1])
  return out


def tpu_sparse_dense_matmul_grad(activation_gradients, preprocessed_inputs,
                                 embedding_variables, feature_specs, *,
                                 global_device_count: int | None = None,
                                 sharding_strategy: str = "MOD",
                                 label: str = "", step=None,
                                 num_sc_per_device: int | None = None,
                                 enable_minibatching: bool = False,
                                 perform_stacking: bool = True,
                                 use_gradient_stacking_primitive=False,
                                 embedding_var_limits=None):
  """Backward pass + optimizer update (embedding.py:1297-1529).

  Returns the updated variables per stacked table, in the structure each
  was given in (EmbeddingVariables or a (table, *slots) tuple); the tensors
  are updated in place.
  """
  if isinstance(preprocessed_inputs, SparseDenseMatmulInput):
    warnings.warn("SparseDenseMatmulInput is deprecated. Please use "
                  "PreprocessedInput instead.", DeprecationWarning)
    preprocessed_inputs = PreprocessedInput(preprocessed_inputs)
  rp, eid, sid, gains = preprocessed_inputs.sparse_dense_matmul_input
  assert rp.keys() == embedding_variables.keys()
  stacked = get_stacked_table_specs(feature_specs)
  assert rp.keys() == stacked.keys()
  num_sc_per_device = _get_num_sc_per_device(num_sc_per_device)
  if perform_stacking:
    _assert_same_structure(feature_specs, activation_gradients,
                           "feature_specs", "activation_gradients")
    # Gradient stacking fused into the kernel: each stack's update reads the
    # per-feature gradients in place (stack_embedding_gradients copies them
    # into one matrix; it remains the path for stacks with too many blocks).
    by_stack = collections.defaultdict(list)
    for g, fs in zip(_tree.tree_leaves(activation_gradients),
                     _tree.tree_leaves(feature_specs)):
      if fs._id_transformation is None:  # pylint: disable=protected-access
        raise ValueError("FeatureIdTransformation cannot be None here. It is "
                         f"None for {fs.name}")
      by_stack[fs.table_spec.stacked_table_spec.stack_name].append((fs, g))
    grads = {}
    for name, items in by_stack.items():
      items.sort(key=lambda x: x[0].id_transformation.row_offset)
      ev = embedding_variables[name]
      table = ev.table if isinstance(ev, EmbeddingVariables) else ev[0]
      blocks = None
      if (not use_gradient_stacking_primitive and
          len(getattr(table, "shape", ())) == 2):
        blocks = _gradient_blocks(
            stacked[name], items, num_sc_per_device,
            (getattr(preprocessed_inputs, "csr_num_entries", None) or
             {}).get(name))
      if blocks is None:
        blocks = stack_embedding_gradients(
            [g for _, g in items], [fs for fs, _ in items],
            num_sc_per_device, global_device_count,
            use_gradient_stacking_primitive)[name]
      grads[name] = blocks
  else:
    grads = activation_gradients
  assert rp.keys() == grads.keys()
  strategy = int(sharding_strategy_to_enum(sharding_strategy))
  nmb = _resolve_scalar_minibatches(preprocessed_inputs.num_minibatches)
  g_count = 1 if global_device_count is None else global_device_count
  def update(name):
    spec = stacked[name]
    ev = embedding_variables[name]
    opt = spec.optimizer
    hyper = opt.get_hyperparameters(step)
    symbol = f"{opt.short_name()}-{spec.stack_name}{label}"
    kwargs = {}
    if isinstance(opt, embedding_spec.FTRLOptimizerSpec):
      kwargs["multiply_linear_by_learning_rate"] = (
          opt.multiply_linear_by_learning_rate)
    if embedding_var_limits is not None:
      kwargs["min_value"], kwargs["max_value"] = embedding_var_limits[name]
    flat, treedef = _tree.tree_flatten(ev)
    extra = dict(
        num_sc_per_device=num_sc_per_device, global_device_count=g_count,
        csr_sorted_by_row=getattr(preprocessed_inputs, "csr_sorted_by_row",
                                  None),
        csr_num_entries=(getattr(preprocessed_inputs, "csr_num_entries",
                                 None) or {}).get(name))
    if isinstance(opt, embedding_spec.CustomOptimizerSpec):
      # The update as StableHLO text, clipped to the limits
      # (embedding.py:1441-1495); operands in the custom primitive's order.
      limits = (embedding_var_limits or {}).get(name, (None, None))
      text = _custom_update_text(
          opt, spec.stack_embedding_dim,
          len(opt.slot_variables_initializers()), len(hyper), *limits)
      res = opt.get_optimizer_primitive().bind(
          rp[name], eid[name], sid[name], gains[name], nmb, grads[name],
          *hyper, *flat, num_hyperparameters=len(hyper), stablehlo=text,
          max_ids_per_partition=spec.max_ids_per_partition,
          max_unique_ids_per_partition=spec.max_unique_ids_per_partition,
          computation_name=symbol, sharding_strategy=strategy,
          enable_minibatching=enable_minibatching, **extra)
    else:
      res = opt.get_optimizer_primitive().bind(
          rp[name], eid[name], sid[name], gains[name], nmb, *flat,
          grads[name], *hyper,
          max_ids_per_partition=spec.max_ids_per_partition,
          max_unique_ids_per_partition=spec.max_unique_ids_per_partition,
          computation_name=symbol, sharding_strategy=strategy,
          enable_minibatching=enable_minibatching, **extra, **kwargs)
    res = res if isinstance(res, tuple) else (res,)
    # The updated variables in the structure they came in
    # (embedding.py:1524-1527): EmbeddingVariables stay EmbeddingVariables
    # (with their slot type), a plain (table, *slots) tuple stays a tuple.
    return _tree.tree_unflatten(treedef, list(res))

  # Independent stacks of different widths update concurrently.
  results = _native.run_per_stack(
      stacked.keys(), update, lambda n: stacked[n].stack_embedding_dim)
  return {name: results[name] for name in stacked}


@functools.lru_cache(maxsize=64)
def _custom_text(fn, stablehlo, dim, num_slots, num_hyper, lo, hi):
  if stablehlo is not None:
    return custom_optimizer_lowering.wrap_stablehlo_with_limits(
        stablehlo, dim, num_slots, num_hyper, lo, hi)
  return custom_optimizer_lowering.lower_to_stablehlo(
      fn, dim, num_slots, num_hyper, lo, hi)


def _custom_update_text(opt, dim, num_slots, num_hyper, lo, hi) -> str:
  """StableHLO text of a CustomOptimizerSpec's update (cached per spec
  contents)."""
  if opt.stablehlo is None and opt.custom_computation_fn is None:
    raise ValueError("Either stablehlo or custom_computation_fn must be "
                     "provided for CustomOptimizerSpec")
  stablehlo = opt.stablehlo
  if isinstance(stablehlo, bytes):
    stablehlo = stablehlo.decode("utf-8")
  return _custom_text(opt.custom_computation_fn if stablehlo is None else
                      None, stablehlo, int(dim), num_slots, num_hyper,
                      None if lo is None else float(lo),
                      None if hi is None else float(hi))


def init_embedding_variables(rng, table_specs, global_sharding=None,
                             num_sparsecore_per_device: int | None = None,
                             bypass_mesh_check: bool = False):
  """Allocates every stacked table and its slots on the GPU.

  `rng` is a seed or a torch.Generator. Each table's rows are initialised by
  its initializer per SparseCore shard and laid out like the reference
  (embedding.py:1532-1591): for shard s, the tables of the stack in
  row_offset_in_shard order.
  """
  del global_sharding, bypass_mesh_check
  t = _native.require_gpu()
  dev = _native.device()
  s_count = _get_num_sc_per_device(num_sparsecore_per_device)
  if isinstance(rng, int):
    gen = t.Generator(device=dev)
    gen.manual_seed(rng)
  else:
    gen = rng
  stacks = collections.defaultdict(list)
  for ts in _tree.tree_leaves(table_specs):
    stacks[ts.setting_in_stack.stack_name].append(ts)
  out = {}
  for name, specs in stacks.items():
    specs.sort(key=lambda x: x.setting_in_stack.row_offset_in_shard)
    dim = specs[0].setting_in_stack.padded_embedding_dim
    tables, slots = [], None
    for _ in range(s_count):
      for ts in specs:
        rows = ts.setting_in_stack.padded_vocab_size // s_count
        init = ts.initializer or embedding_spec.zeros
        tables.append(init(gen, (rows, dim), device=dev))
        slot_inits = ts.optimizer.slot_variables_initializers()
        vals = [si(gen, (rows, dim), device=dev) for si in slot_inits]
        slots = [[] for _ in vals] if slots is None else slots
        for k, v in enumerate(vals):
          slots[k].append(v)
    table = t.cat(tables, dim=0)
    slot_vals = tuple(t.cat(s, dim=0) for s in (slots or []))
    slot_type = type(specs[0].optimizer.slot_variables_initializers())
    if hasattr(slot_type, "_fields"):  # the optimizer's *SlotVariables
      slot_vals = slot_type(*slot_vals)
    out[name] = EmbeddingVariables(table, slot_vals)
  return out


def update_preprocessing_parameters(feature_specs, updated_params,
                                    num_sc_per_device: int) -> None:
  """Writes observed limits / buffer sizes into the StackedTableSpecs."""

  def update(fs):
    st = fs.table_spec.stacked_table_spec
    name = st.stack_name
    max_ids = updated_params.max_ids_per_partition.get(
        name, st.max_ids_per_partition)
    max_unique = updated_params.max_unique_ids_per_partition.get(
        name, st.max_unique_ids_per_partition)
    size = updated_params.get_required_buffer_size_per_device(
        name, num_sc_per_device)
    if size is None:
      size = st.suggested_coo_buffer_size_per_device
    fs.table_spec.stacked_table_spec = dataclasses.replace(
        st, max_ids_per_partition=int(np.max(max_ids)),
        max_unique_ids_per_partition=int(np.max(max_unique)),
        suggested_coo_buffer_size_per_device=size)

  for fs in _tree.tree_leaves(feature_specs):
    update(fs)


# Spec <-> proto conversion, re-exported as the reference does
# (embedding.py:1759-1765).
from jax_tpu_embedding.sparsecore.lib.nn import embedding_proto_utils  # pylint: disable=g-import-not-at-top,g-bad-import-order

get_optimizer_class = embedding_proto_utils.get_optimizer_class
get_optimizer_type = embedding_proto_utils.get_optimizer_type
optimizer_spec_to_proto = embedding_proto_utils.optimizer_spec_to_proto
proto_to_optimizer_spec = embedding_proto_utils.proto_to_optimizer_spec
create_proto_from_feature_specs = (
    embedding_proto_utils.create_proto_from_feature_specs)
