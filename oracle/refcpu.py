"""ctypes front end of the CPU oracle (``oracle/refcpu.cc``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, always as the checker. The
product package never imports it.

Besides thin wrappers over the C stages, this module restates the two pieces of
host logic the reference keeps in its pybind layer, so the oracle can be driven
from the same feature specs as the product:

* ``stacked_table_metadata`` follows ``GetStackedTableMetadata``
  (``lib/core/pybind_input_preprocessing.cc:55-122``): one record per feature,
  grouped by ``setting_in_stack.stack_name`` and ordered by ``row_offset``.
* ``preprocess`` follows ``PyPreprocessSparseDenseMatmulInput``
  (``pybind_input_preprocessing.cc:124-188``) and
  ``PreprocessSparseDenseMatmulInput`` (``input_preprocessing.cc:800-959``),
  with minibatching on a single host.

``sparse_dense_matmul_grad_custom`` restates the custom-optimizer update
(``lib/core/primitives/sparse_dense_matmul_optimizer_grad.py``; the test-side
expectation of ``primitives/tests/sparse_dense_matmul_optimizer_grad_test.py:81-140``):
per-row gradient sums from the C backward, then the user's function in numpy
float32 on the touched rows. It is pinned by equality with the oracle's
built-in SGD and Adagrad (bit for bit) and by the reference's custom-Adagrad
literal table (``tpu_sparse_dense_matmul_grad_test.py:1324-1486``), in
``tests/test_custom_optimizer.py``.
"""

from __future__ import annotations

import ctypes
import dataclasses
import os
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "librefcpu.so"

COMBINERS = {"sum": 0, "mean": 1, "sqrtn": 2}


class RefFeature(ctypes.Structure):
  _fields_ = [
      ("ids", ctypes.c_void_p),
      ("row_splits", ctypes.c_void_p),
      ("weights", ctypes.c_void_p),
      ("num_rows", ctypes.c_int64),
      ("row_offset", ctypes.c_int32),
      ("col_offset", ctypes.c_int32),
      ("col_shift", ctypes.c_int32),
      ("pad_", ctypes.c_int32),
  ]


_lib = None


def lib() -> ctypes.CDLL:
  """Loads the oracle library, building it with make when it is missing."""
  global _lib
  if _lib is not None:
    return _lib
  if not _LIB_PATH.exists():
    import subprocess  # pylint: disable=g-import-not-at-top

    subprocess.check_call(["make", "-s", "-C", str(_HERE)])
  l = ctypes.CDLL(str(_LIB_PATH))
  vp, i32, i64, f32 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                       ctypes.c_float)
  l.ref_get_col_id.argtypes = [i32, i32, i32, i32]
  l.ref_get_col_id.restype = i32
  l.ref_grouping_key.argtypes = [ctypes.c_uint32, ctypes.c_uint32, i32]
  l.ref_grouping_key.restype = ctypes.c_uint64
  l.ref_col_id_from_key.argtypes = [ctypes.c_uint64, i32]
  l.ref_col_id_from_key.restype = ctypes.c_uint32
  l.ref_data_from_key.argtypes = [ctypes.c_uint64]
  l.ref_data_from_key.restype = ctypes.c_uint32
  l.ref_extract_slice.argtypes = [vp, i32, i32, i32, i32, i32, i32, i32, vp,
                                  vp, vp, vp]
  l.ref_extract_device.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp,
                                   vp, vp, vp]
  l.ref_sort_and_group.argtypes = [i32, vp, vp, vp, vp, i32, i32, i32, i32,
                                   i32, vp, vp, vp, vp, vp, vp, vp, vp]
  l.ref_fill_device.argtypes = [i32, vp, vp, vp, vp, i32, i32, i64, i32, vp,
                                vp, vp, vp, vp]
  l.ref_preprocess_stack.argtypes = [vp, i32, i32, i32, i32, i32, i32, i32,
                                     i32, i32, i64, vp, vp, vp, vp, vp, vp, vp,
                                     vp]
  l.ref_theoretical_max_coo_buffer_size.argtypes = [i32, i32, i32]
  l.ref_theoretical_max_coo_buffer_size.restype = i64
  l.ref_coo_buffer_size_per_device.argtypes = [i32, i64, i32, i32]
  l.ref_coo_buffer_size_per_device.restype = i64
  l.ref_theoretical_max_coo_buffer_size_ex.argtypes = [i32, i32, i32, i32]
  l.ref_theoretical_max_coo_buffer_size_ex.restype = i64
  l.ref_coo_buffer_size_per_device_ex.argtypes = [i32, i64, i32, i32, i32]
  l.ref_coo_buffer_size_per_device_ex.restype = i64
  l.ref_sparse_dense_matmul.argtypes = [vp, vp, vp, vp, i64, i32, i32, i32,
                                        i32, vp, i64, i32, vp, i64, i32]
  l.ref_sparse_dense_matmul_grad.argtypes = [vp, vp, vp, vp, i64, i32, i32,
                                             i32, i32, vp, i64, vp, vp, i64,
                                             i32, i32, f32, i32, f32, f32, i32]
  l.ref_sparse_dense_matmul_grad_optimizer.argtypes = [
      vp, vp, vp, vp, i64, i32, i32, i32, i32, vp, i64, vp, vp, vp, i64, i32,
      i32, vp, i32, i32, f32, f32, i32]
  u32, u64 = ctypes.c_uint32, ctypes.c_uint64
  l.ref_minibatching_bucket.argtypes = [i32]
  l.ref_minibatching_bucket.restype = u32
  l.ref_highway_hash64.argtypes = [vp, i64, vp]
  l.ref_highway_hash64.restype = u64
  l.ref_compute_minibatching_split.argtypes = [vp, i32, i32]
  l.ref_compute_minibatching_split.restype = u64
  l.ref_merge_buckets.argtypes = [u64, i32, vp]
  l.ref_merge_partitioned.argtypes = [i32, vp, vp, vp, vp, i32, u64, vp]
  l.ref_preprocess_stack_minibatching.argtypes = [
      vp, i32, i32, i32, i32, i32, i32, i32, i32, i32, i64, i32, u64, vp, vp,
      vp, vp, vp, vp, vp, vp, vp]
  for fn in ("ref_extract_slice", "ref_extract_device", "ref_sort_and_group",
             "ref_fill_device", "ref_preprocess_stack",
             "ref_sparse_dense_matmul", "ref_sparse_dense_matmul_grad",
             "ref_sparse_dense_matmul_grad_optimizer", "ref_merge_buckets",
             "ref_merge_partitioned", "ref_preprocess_stack_minibatching"):
    getattr(l, fn).restype = i32
  _lib = l
  return l


def _p(a: np.ndarray | None):
  return None if a is None else a.ctypes.data


# ---------------------------------------------------------------------------
# Stage wrappers.
# ---------------------------------------------------------------------------


def get_col_id(embedding_id, col_shift, col_offset, num_scs_mod) -> int:
  return lib().ref_get_col_id(embedding_id, col_shift, col_offset, num_scs_mod)


def grouping_key(col_id, data, num_scs_bit) -> int:
  return lib().ref_grouping_key(col_id, data, num_scs_bit)


def col_id_from_key(key, num_scs_bit) -> int:
  return lib().ref_col_id_from_key(key, num_scs_bit)


def data_from_key(key) -> int:
  return lib().ref_data_from_key(key)


# Minibatching (coo_format.h:31-49, minibatching_splits_impl.h,
# partitioned_coo_tensors.h:157-215).
MAX_MINIBATCHING_BUCKETS = 64


def highway_hash64(data: bytes, key) -> int:
  buf = np.frombuffer(bytes(data), np.uint8) if data else np.zeros(1, np.uint8)
  k = np.ascontiguousarray(np.asarray(key, np.uint64))
  return int(lib().ref_highway_hash64(_p(buf), len(data), _p(k)))


def minibatching_bucket(col_id) -> int:
  return int(lib().ref_minibatching_bucket(int(col_id)))


def compute_minibatching_split(values, max_value) -> tuple[int, np.ndarray]:
  """ComputeMinibatchingSplit: (split bits, the values as it leaves them)."""
  v = np.array(values, np.int32)
  return int(lib().ref_compute_minibatching_split(_p(v), len(v),
                                                  int(max_value))), v


def merge_buckets(split, n) -> list[tuple[int, int]]:
  """MergeBuckets<n>: the merged (left, right) bucket pairs in call order."""
  pairs = np.zeros(2 * n, np.int32)
  k = lib().ref_merge_buckets(int(split), int(n), _p(pairs))
  return [(int(pairs[2 * i]), int(pairs[2 * i + 1])) for i in range(k)]


def merge_partitioned(buckets, num_scs, split):
  """PartitionedCooTensors::Merge<len(buckets)>: `buckets` is a list of
  lists of (row, col, gain); returns the list of minibatches (lists of
  (row, col, gain))."""
  sizes = np.array([len(b) for b in buckets], np.int32)
  flat = [c for b in buckets for c in b] or [(0, 0, 0.0)]
  rows = np.array([c[0] for c in flat], np.int32)
  cols = np.array([c[1] for c in flat], np.int32)
  gains = np.array([c[2] for c in flat], np.float32)
  offsets = np.zeros(len(buckets) + 1, np.int32)
  n = lib().ref_merge_partitioned(len(buckets), _p(sizes), _p(rows), _p(cols),
                                  _p(gains), int(num_scs), int(split),
                                  _p(offsets))
  return [[(int(rows[i]), int(cols[i]), float(gains[i]))
           for i in range(offsets[m], offsets[m + 1])] for m in range(n)]


@dataclasses.dataclass
class RaggedFeature:
  """Values + row splits (+ optional weights) of one feature batch."""

  ids: np.ndarray
  row_splits: np.ndarray
  weights: np.ndarray | None = None
  row_offset: int = 0
  col_offset: int = 0
  col_shift: int = 0

  def __post_init__(self):
    self.ids = np.ascontiguousarray(self.ids, dtype=np.int32)
    self.row_splits = np.ascontiguousarray(self.row_splits, dtype=np.int64)
    if self.weights is not None:
      self.weights = np.ascontiguousarray(self.weights, dtype=np.float32)

  @property
  def num_rows(self) -> int:
    return len(self.row_splits) - 1

  def as_struct(self) -> RefFeature:
    return RefFeature(_p(self.ids), _p(self.row_splits), _p(self.weights),
                      self.num_rows, self.row_offset, self.col_offset,
                      self.col_shift, 0)


def ragged_from_rows(rows, weights=None, **kw) -> RaggedFeature:
  """Builds a RaggedFeature from a list of per-sample id sequences."""
  lens = [len(r) for r in rows]
  splits = np.zeros(len(rows) + 1, np.int64)
  splits[1:] = np.cumsum(lens)
  ids = (np.concatenate([np.asarray(r, np.int64) for r in rows])
         if rows and sum(lens) else np.zeros(0, np.int64)).astype(np.int32)
  w = None
  if weights is not None:
    w = (np.concatenate([np.asarray(x, np.float32) for x in weights])
         if sum(lens) else np.zeros(0, np.float32))
  return RaggedFeature(ids, splits, w, **kw)


def ragged_from_array(feature, weights=None, **kw) -> RaggedFeature:
  """Converts a 2-D array, a 1-D object array of rows, or a ragged object
  with flat `values` and `row_splits` to RaggedFeature."""
  if hasattr(feature, "values") and hasattr(feature, "row_splits"):
    w = None
    if weights is not None:
      w = np.asarray(getattr(weights, "values", weights),
                     np.float32).reshape(-1)
    return RaggedFeature(np.asarray(feature.values, np.int32).reshape(-1),
                         np.asarray(feature.row_splits, np.int64), w, **kw)
  feature = np.asarray(feature) if not isinstance(feature, list) else feature
  if isinstance(feature, np.ndarray) and feature.ndim == 2 and \
      feature.dtype != object:
    b, k = feature.shape
    splits = np.arange(b + 1, dtype=np.int64) * k
    w = None if weights is None else np.asarray(weights,
                                                np.float32).reshape(-1)
    return RaggedFeature(feature.reshape(-1), splits, w, **kw)
  rows = list(feature)
  wrows = None if weights is None else list(weights)
  return ragged_from_rows(rows, wrows, **kw)


def extract_slice(feature: RaggedFeature, slice_start, slice_end, row_offset,
                  col_offset, col_shift, num_scs, combiner="sum"):
  """One ExtractCooTensors call; returns (rows, cols, gains)."""
  n = int(feature.row_splits[slice_end] - feature.row_splits[slice_start])
  rows = np.zeros(n, np.int32)
  cols = np.zeros(n, np.int32)
  gains = np.zeros(n, np.float32)
  count = ctypes.c_int64(0)
  st = feature.as_struct()
  lib().ref_extract_slice(ctypes.byref(st), slice_start, slice_end, row_offset,
                          col_offset, col_shift, num_scs,
                          COMBINERS[combiner], _p(rows), _p(cols), _p(gains),
                          ctypes.byref(count))
  return rows, cols, gains


def extract_device(features, local_device_id, local_device_count,
                   global_device_count, num_sc_per_device, combiner="sum"):
  """ExtractCooTensorsForAllFeaturesPerLocalDevice.

  Returns (rows, cols, gains, sc_sizes, batch_size_for_device).
  """
  total = sum(int(f.row_splits[-1]) for f in features)
  structs = (RefFeature * len(features))(*[f.as_struct() for f in features])
  rows = np.zeros(max(total, 1), np.int32)
  cols = np.zeros(max(total, 1), np.int32)
  gains = np.zeros(max(total, 1), np.float32)
  sizes = np.zeros(num_sc_per_device, np.int64)
  bfd = ctypes.c_int32(0)
  st = lib().ref_extract_device(structs, len(features), local_device_id,
                                local_device_count, global_device_count,
                                num_sc_per_device, COMBINERS[combiner],
                                _p(rows), _p(cols), _p(gains), _p(sizes),
                                ctypes.byref(bfd))
  if st != 0:
    raise ValueError("invalid batch split for the number of SparseCores")
  n = int(sizes.sum())
  return rows[:n], cols[:n], gains[:n], sizes, int(bfd.value)


@dataclasses.dataclass
class GroupResult:
  per_sc: list  # list of (rows, cols, gains) arrays per local SC
  max_ids_per_partition: np.ndarray
  max_unique_ids_per_partition: np.ndarray
  required_buffer_size: np.ndarray
  dropped_id_count: int
  limit_exceeded: bool


def sort_and_group(rows, cols, gains, sc_sizes, *, num_scs,
                   max_ids_per_partition, max_unique_ids_per_partition,
                   allow_id_dropping=False, has_variable_weights=None):
  """SortAndGroupCooTensorsPerLocalDevice (no minibatching)."""
  rows = np.ascontiguousarray(rows, np.int32)
  cols = np.ascontiguousarray(cols, np.int32)
  gains = np.ascontiguousarray(gains, np.float32)
  sc_sizes = np.ascontiguousarray(sc_sizes, np.int64)
  if has_variable_weights is None:
    has_variable_weights = bool(np.any(gains != 1.0))
  s_count = len(sc_sizes)
  n = max(len(rows), 1)
  g_rows = np.zeros(n, np.int32)
  g_cols = np.zeros(n, np.int32)
  g_gains = np.zeros(n, np.float32)
  g_sizes = np.zeros(s_count, np.int64)
  max_ids = np.zeros(num_scs, np.int32)
  max_unique = np.zeros(num_scs, np.int32)
  required = np.zeros(s_count, np.int32)
  dropped = ctypes.c_int64(0)
  st = lib().ref_sort_and_group(s_count, _p(sc_sizes), _p(rows), _p(cols),
                                _p(gains), int(has_variable_weights), num_scs,
                                max_ids_per_partition,
                                max_unique_ids_per_partition,
                                int(allow_id_dropping), _p(g_rows), _p(g_cols),
                                _p(g_gains), _p(g_sizes), _p(max_ids),
                                _p(max_unique), _p(required),
                                ctypes.byref(dropped))
  per_sc = []
  base = 0
  for s in range(s_count):
    k = int(g_sizes[s])
    per_sc.append((g_rows[base:base + k].copy(), g_cols[base:base + k].copy(),
                   g_gains[base:base + k].copy()))
    base += k
  return GroupResult(per_sc, max_ids, max_unique, required,
                     int(dropped.value), st == 2)


def fill_device(per_sc, *, num_scs, batch_size_per_sc, coo_size, rp_per_sc,
                fill_value=None):
  """FillLocalDeviceBuffer; unwritten slots keep ``fill_value`` sentinels."""
  s_count = len(per_sc)
  g_sizes = np.array([len(x[0]) for x in per_sc], np.int64)
  stride = [0]
  g_rows = np.concatenate([x[0] for x in per_sc] + [np.zeros(1, np.int32)])
  g_cols = np.concatenate([x[1] for x in per_sc] + [np.zeros(1, np.int32)])
  g_gains = np.concatenate([x[2] for x in per_sc] + [np.zeros(1, np.float32)])
  del stride
  sentinel_i = -7 if fill_value is None else fill_value
  rp = np.full(s_count * rp_per_sc, sentinel_i, np.int32)
  eid = np.full(coo_size, sentinel_i, np.int32)
  sid = np.full(coo_size, sentinel_i, np.int32)
  gains = np.full(coo_size, -7.0, np.float32)
  dropped = ctypes.c_int64(0)
  # ref_fill_device reads the grouped lists SC after SC, packed.
  lib().ref_fill_device(s_count, _p(g_sizes), _p(g_rows), _p(g_cols),
                        _p(g_gains), num_scs, batch_size_per_sc, coo_size,
                        rp_per_sc, _p(rp), _p(eid), _p(sid), _p(gains),
                        ctypes.byref(dropped))
  return rp, eid, sid, gains, int(dropped.value)


# ---------------------------------------------------------------------------
# Spec-driven entry point (pybind_input_preprocessing.cc restated).
# ---------------------------------------------------------------------------


@dataclasses.dataclass
class FeatureMetadata:
  name: str
  feature_index: int
  max_ids_per_partition: int
  max_unique_ids_per_partition: int
  row_offset: int
  col_offset: int
  col_shift: int
  batch_size: int
  suggested_coo_buffer_size_per_device: int | None
  combiner: str


def stacked_table_metadata(feature_specs) -> dict[str, list[FeatureMetadata]]:
  """GetStackedTableMetadata (pybind_input_preprocessing.cc:55-122)."""
  out: dict[str, list[FeatureMetadata]] = {}
  for i, fs in enumerate(feature_specs):
    t = fs.table_spec
    st = t.stacked_table_spec
    stack_name = t.setting_in_stack.stack_name
    tr = fs._id_transformation  # pylint: disable=protected-access
    row_offset = col_offset = col_shift = 0
    if tr is not None:
      row_offset, col_offset, col_shift = (tr.row_offset, tr.col_offset,
                                           tr.col_shift)
    out.setdefault(stack_name, []).append(
        FeatureMetadata(fs.name, i, st.max_ids_per_partition,
                        st.max_unique_ids_per_partition, row_offset,
                        col_offset, col_shift, int(fs.input_shape[0]),
                        st.suggested_coo_buffer_size_per_device, st.combiner))
  for v in out.values():
    v.sort(key=lambda m: m.row_offset)
  return out


@dataclasses.dataclass
class PreprocessResult:
  row_pointers: dict
  embedding_ids: dict
  sample_ids: dict
  gains: dict
  max_ids_per_partition: dict
  max_unique_ids_per_partition: dict
  required_buffer_sizes: dict
  dropped_id_count: dict
  num_minibatches: int = 1


def preprocess(features, features_weights, feature_specs, local_device_count,
               global_device_count, *, num_sc_per_device,
               has_leading_dimension=False, allow_id_dropping=False,
               fill_value=0, enable_minibatching=False):
  """CPU preprocessing of a list of features.

  With `enable_minibatching` (single host), the passes of
  PreprocessSparseDenseMatmulInput (input_preprocessing.cc:852-957): a first
  pass over every stack; if one of them exceeds a limit, a bucket pass over
  every stack whose splits are OR-ed into one, and a second fill with that
  many minibatches. Row pointers then have 64 * S * max(NS, 8) entries per
  device.

  Raises ValueError on invalid options and RuntimeError where the reference
  aborts (limits exceeded with dropping disabled).
  """
  if enable_minibatching:
    return _preprocess_minibatching(
        features, features_weights, feature_specs, local_device_count,
        global_device_count, num_sc_per_device=num_sc_per_device,
        has_leading_dimension=has_leading_dimension,
        allow_id_dropping=allow_id_dropping, fill_value=fill_value)
  L, G, S = local_device_count, global_device_count, num_sc_per_device
  if L <= 0 or G <= 0 or S <= 0 or G < L:
    raise ValueError("invalid device counts")
  ns = S * G
  if ns & (ns - 1):
    raise ValueError(f"Total number of SparseCores ({ns}) must be a power of 2.")
  rp_per_sc = max(ns, 8)
  stacks = stacked_table_metadata(feature_specs)
  res = PreprocessResult({}, {}, {}, {}, {}, {}, {}, {})
  for stack_name, metas in stacks.items():
    ragged = []
    for m in metas:
      w = None if features_weights is None else \
          features_weights[m.feature_index]
      ragged.append(ragged_from_array(features[m.feature_index], w,
                                      row_offset=m.row_offset,
                                      col_offset=m.col_offset,
                                      col_shift=m.col_shift))
    b_dev = sum(f.num_rows // L for f in ragged)
    if b_dev > (1 << 26) - 1:
      raise ValueError("local batch size exceeds the CooFormat key limit")
    has_w = features_weights is not None
    c = lib().ref_coo_buffer_size_per_device(
        metas[0].max_ids_per_partition,
        metas[0].suggested_coo_buffer_size_per_device or 0, G, S)
    if c < 0:
      raise RuntimeError("Suggested Coo Buffer Size is larger than the "
                         "theoretical max")
    structs = (RefFeature * len(ragged))(*[f.as_struct() for f in ragged])
    rp = np.full(L * S * rp_per_sc, fill_value, np.int32)
    eid = np.full(L * c, fill_value, np.int32)
    sid = np.full(L * c, fill_value, np.int32)
    gains = np.full(L * c, fill_value, np.float32)
    max_ids = np.zeros(L * ns, np.int32)
    max_unique = np.zeros(L * ns, np.int32)
    required = np.zeros(L * S, np.int32)
    dropped = ctypes.c_int64(0)
    st = lib().ref_preprocess_stack(
        structs, len(ragged), L, G, S, COMBINERS[metas[0].combiner],
        int(has_w), metas[0].max_ids_per_partition,
        metas[0].max_unique_ids_per_partition, int(allow_id_dropping), c,
        _p(rp), _p(eid), _p(sid), _p(gains), _p(max_ids), _p(max_unique),
        _p(required), ctypes.byref(dropped))
    if st == 1:
      raise ValueError("batch size not divisible by num_sc_per_device")
    if st == 2:
      raise RuntimeError(f"Observed max ids per partition exceeds the limit "
                         f"for table: {stack_name}")
    if has_leading_dimension:
      rp, eid, sid, gains = (rp.reshape(L, -1), eid.reshape(L, -1),
                             sid.reshape(L, -1), gains.reshape(L, -1))
    res.row_pointers[stack_name] = rp
    res.embedding_ids[stack_name] = eid
    res.sample_ids[stack_name] = sid
    res.gains[stack_name] = gains
    res.max_ids_per_partition[stack_name] = max_ids
    res.max_unique_ids_per_partition[stack_name] = max_unique
    res.required_buffer_sizes[stack_name] = required
    res.dropped_id_count[stack_name] = int(dropped.value)
  return res


def _preprocess_minibatching(features, features_weights, feature_specs,
                             local_device_count, global_device_count, *,
                             num_sc_per_device, has_leading_dimension,
                             allow_id_dropping, fill_value):
  L, G, S = local_device_count, global_device_count, num_sc_per_device
  if L <= 0 or G <= 0 or S <= 0 or G < L:
    raise ValueError("invalid device counts")
  ns = S * G
  if ns & (ns - 1):
    raise ValueError(f"Total number of SparseCores ({ns}) must be a power of 2.")
  rpb = max(ns, 8)
  stacks = stacked_table_metadata(feature_specs)
  has_w = features_weights is not None
  res = PreprocessResult({}, {}, {}, {}, {}, {}, {}, {})
  state = {}
  for stack_name, metas in stacks.items():
    ragged = []
    for m in metas:
      w = None if features_weights is None else \
          features_weights[m.feature_index]
      ragged.append(ragged_from_array(features[m.feature_index], w,
                                      row_offset=m.row_offset,
                                      col_offset=m.col_offset,
                                      col_shift=m.col_shift))
    c = lib().ref_coo_buffer_size_per_device_ex(
        metas[0].max_ids_per_partition,
        metas[0].suggested_coo_buffer_size_per_device or 0, G, S, 1)
    if c < 0:
      raise RuntimeError("Suggested Coo Buffer Size is larger than the "
                         "theoretical max")
    structs = (RefFeature * len(ragged))(*[f.as_struct() for f in ragged])
    bufs = dict(
        rp=np.full(L * S * MAX_MINIBATCHING_BUCKETS * rpb, fill_value,
                   np.int32),
        eid=np.full(L * c, fill_value, np.int32),
        sid=np.full(L * c, fill_value, np.int32),
        gains=np.full(L * c, fill_value, np.float32),
        max_ids=np.zeros(L * ns, np.int32),
        max_unique=np.zeros(L * ns, np.int32),
        required=np.zeros(L * S, np.int32))
    state[stack_name] = (metas, ragged, structs, c, bufs)

  def run(stack_name, stage, split=0):
    metas, ragged, structs, c, b = state[stack_name]
    dropped = ctypes.c_int64(0)
    flag = ctypes.c_uint64(0)
    st = lib().ref_preprocess_stack_minibatching(
        structs, len(ragged), L, G, S, COMBINERS[metas[0].combiner],
        int(has_w), metas[0].max_ids_per_partition,
        metas[0].max_unique_ids_per_partition, int(allow_id_dropping), c,
        stage, split, _p(b["rp"]), _p(b["eid"]), _p(b["sid"]),
        _p(b["gains"]), _p(b["max_ids"]), _p(b["max_unique"]),
        _p(b["required"]), ctypes.byref(dropped), ctypes.byref(flag))
    if st == 1:
      raise ValueError("batch size not divisible by num_sc_per_device")
    if st == 2:
      raise RuntimeError(f"Observed max ids per partition exceeds the limit "
                         f"for table: {stack_name}")
    return int(dropped.value), int(flag.value)

  dropped, required = {}, False
  for name in state:
    dropped[name], flag = run(name, 0)
    required = required or flag != 0
  split = 0
  if required:
    for name in state:
      split |= run(name, 1)[1]
    for name in state:
      dropped[name] = run(name, 2, split)[0]
  res.num_minibatches = bin(split).count("1") + 1
  for name, (metas, ragged, structs, c, b) in state.items():
    rp, eid, sid, gains = b["rp"], b["eid"], b["sid"], b["gains"]
    if has_leading_dimension:
      rp, eid, sid, gains = (rp.reshape(L, -1), eid.reshape(L, -1),
                             sid.reshape(L, -1), gains.reshape(L, -1))
    res.row_pointers[name] = rp
    res.embedding_ids[name] = eid
    res.sample_ids[name] = sid
    res.gains[name] = gains
    res.max_ids_per_partition[name] = b["max_ids"]
    res.max_unique_ids_per_partition[name] = b["max_unique"]
    res.required_buffer_sizes[name] = b["required"]
    res.dropped_id_count[name] = dropped[name]
  return res


# ---------------------------------------------------------------------------
# Lookup and update oracle.
# ---------------------------------------------------------------------------


def _threads(threads):
  return threads if threads else min(16, os.cpu_count() or 1)


def _rp_per_segment(rp, num_sc_per_device, num_scs, num_minibatches):
  if num_minibatches:
    return max(num_scs, 8)
  return len(rp) // num_sc_per_device


def sparse_dense_matmul(rp, eid, sid, gains, table, batch, *,
                        num_sc_per_device, num_scs, threads=None,
                        num_minibatches=0):
  """Forward: activations[batch, dim] (or [batch] for a 1-D table).

  num_minibatches > 0: the CSR is in the minibatching layout (blocks of
  max(num_scs, 8) row pointers per SC and minibatch from the start of `rp`,
  positions in the whole buffer)."""
  table = np.ascontiguousarray(table, np.float32)
  dim = 1 if table.ndim == 1 else table.shape[1]
  act = np.zeros((batch, dim), np.float32)
  rp, eid, sid, gains = (np.ascontiguousarray(rp, np.int32).reshape(-1),
                         np.ascontiguousarray(eid, np.int32).reshape(-1),
                         np.ascontiguousarray(sid, np.int32).reshape(-1),
                         np.ascontiguousarray(gains, np.float32).reshape(-1))
  lib().ref_sparse_dense_matmul(_p(rp), _p(eid), _p(sid), _p(gains), len(eid),
                                num_sc_per_device, num_scs,
                                _rp_per_segment(rp, num_sc_per_device, num_scs,
                                                num_minibatches),
                                int(num_minibatches), _p(table),
                                table.shape[0], dim, _p(act), batch,
                                _threads(threads))
  return act.reshape(batch) if table.ndim == 1 else act


def sparse_dense_matmul_grad(rp, eid, sid, gains, act_grad, table,
                             accumulator=None, *, learning_rate,
                             num_sc_per_device, num_scs, min_value=None,
                             max_value=None, threads=None, inplace=False,
                             num_minibatches=0):
  """Backward + SGD (accumulator None) or Adagrad.

  Returns updated copies, or updates `table` / `accumulator` (C-contiguous
  float32) in place when `inplace`.
  """
  if inplace:
    assert table.dtype == np.float32 and table.flags.c_contiguous
    acc = accumulator
  else:
    table = np.array(table, np.float32, copy=True, order="C")
    acc = None if accumulator is None else np.array(accumulator, np.float32,
                                                     copy=True, order="C")
  dim = 1 if table.ndim == 1 else table.shape[1]
  act_grad = np.ascontiguousarray(act_grad, np.float32)
  batch = act_grad.shape[0]
  rp, eid, sid, gains = (np.ascontiguousarray(rp, np.int32).reshape(-1),
                         np.ascontiguousarray(eid, np.int32).reshape(-1),
                         np.ascontiguousarray(sid, np.int32).reshape(-1),
                         np.ascontiguousarray(gains, np.float32).reshape(-1))
  clip = (1 if min_value is not None else 0) | (2 if max_value is not None
                                                 else 0)
  lib().ref_sparse_dense_matmul_grad(
      _p(rp), _p(eid), _p(sid), _p(gains), len(eid), num_sc_per_device,
      num_scs, _rp_per_segment(rp, num_sc_per_device, num_scs, num_minibatches),
      int(num_minibatches), _p(act_grad), batch, _p(table), _p(acc), table.shape[0], dim, 0 if acc is None else 1,
      float(learning_rate), clip,
      float(min_value if min_value is not None else 0.0),
      float(max_value if max_value is not None else 0.0), _threads(threads))
  return (table, acc) if acc is not None else table


# Optimizer kinds of ref_sparse_dense_matmul_grad_optimizer.
OPTIMIZERS = {"sgd": 0, "adagrad": 1, "adam": 2, "adagrad_momentum": 3,
              "ftrl": 4, "laprop": 5, "f2a": 6}
OPTIMIZER_SLOTS = {"sgd": 0, "adagrad": 1, "adam": 2, "adagrad_momentum": 2,
                   "ftrl": 2, "laprop": 2, "f2a": 2}


def sparse_dense_matmul_grad_optimizer(rp, eid, sid, gains, act_grad, table,
                                       slots, *, optimizer: str,
                                       hyperparameters, num_sc_per_device,
                                       num_scs, multiply_linear_by_lr=False,
                                       min_value=None, max_value=None,
                                       threads=None, num_minibatches=0):
  """Backward + any optimizer (`optimizer` a key of OPTIMIZERS), on copies.

  `slots` in the order of the optimizer's slot variables, `hyperparameters`
  in the order of the reference primitive's operands. Returns
  (table, *slots).
  """
  n_slots = OPTIMIZER_SLOTS[optimizer]
  assert len(slots) == n_slots, (optimizer, len(slots))
  table = np.array(table, np.float32, copy=True, order="C")
  slots = [np.array(x, np.float32, copy=True, order="C") for x in slots]
  hp = np.zeros(8, np.float32)
  hp[:len(hyperparameters)] = [np.float32(np.asarray(h, np.float32))
                               for h in hyperparameters]
  dim = 1 if table.ndim == 1 else table.shape[1]
  act_grad = np.ascontiguousarray(act_grad, np.float32)
  batch = act_grad.shape[0]
  rp, eid, sid, gains = (np.ascontiguousarray(rp, np.int32).reshape(-1),
                         np.ascontiguousarray(eid, np.int32).reshape(-1),
                         np.ascontiguousarray(sid, np.int32).reshape(-1),
                         np.ascontiguousarray(gains, np.float32).reshape(-1))
  clip = (1 if min_value is not None else 0) | (2 if max_value is not None
                                                 else 0)
  lib().ref_sparse_dense_matmul_grad_optimizer(
      _p(rp), _p(eid), _p(sid), _p(gains), len(eid), num_sc_per_device,
      num_scs, _rp_per_segment(rp, num_sc_per_device, num_scs, num_minibatches),
      int(num_minibatches), _p(act_grad), batch, _p(table),
      _p(slots[0]) if n_slots > 0 else None,
      _p(slots[1]) if n_slots > 1 else None, table.shape[0], dim,
      OPTIMIZERS[optimizer], _p(hp), 1 if multiply_linear_by_lr else 0, clip,
      float(min_value if min_value is not None else 0.0),
      float(max_value if max_value is not None else 0.0), _threads(threads))
  return (table, *slots)


def touched_rows(rp, eid, *, num_sc_per_device, num_scs, table_rows,
                 num_minibatches=0) -> np.ndarray:
  """Table rows the CSR names (entries of every segment and partition up to
  its row pointer; padding and ids outside the table left out)."""
  rp = np.asarray(rp, np.int64).reshape(-1)
  eid = np.asarray(eid, np.int64).reshape(-1)
  rows_per_part = table_rows // num_scs
  per_seg = len(eid) // num_sc_per_device
  rp_per = _rp_per_segment(rp, num_sc_per_device, num_scs, num_minibatches)
  out = np.zeros(table_rows, bool)
  blocks = (num_sc_per_device * (num_minibatches or 1))
  for blk in range(blocks):
    seg = blk // (num_minibatches or 1)
    base = 0 if num_minibatches else seg * per_seg
    start = 0 if not num_minibatches or blk == 0 else None
    for p in range(num_scs):
      end = int(rp[blk * rp_per + p])
      if start is None:
        prev = int(rp[blk * rp_per - rp_per + num_scs - 1])
        start = (prev + 7) // 8 * 8
      lo, hi = base + start, base + min(end, per_seg if not num_minibatches
                                        else len(eid))
      ids = eid[lo:hi]
      ids = ids[(ids >= 0) & (ids < rows_per_part)]
      out[p * rows_per_part + ids] = True
      start = (end + 7) // 8 * 8
  return out


def sparse_dense_matmul_grad_custom(rp, eid, sid, gains, act_grad, table,
                                    slots, *, update_fn, hyperparameters,
                                    num_sc_per_device, num_scs,
                                    min_value=None, max_value=None,
                                    threads=None):
  """Backward + a custom update: each touched row's gradient summed by the C
  oracle (its SGD with learning rate -1 on a zero table returns the sums),
  then `update_fn(grad, table, *slots, *hyperparameters)` evaluated in numpy
  float32 on the touched rows, then the clipping of the table. Returns
  (table, *slots)."""
  table = np.array(table, np.float32, copy=True)
  slots = [np.array(x, np.float32, copy=True) for x in slots]
  sums = sparse_dense_matmul_grad(rp, eid, sid, gains, act_grad,
                                  np.zeros_like(table), learning_rate=-1.0,
                                  num_sc_per_device=num_sc_per_device,
                                  num_scs=num_scs, threads=threads)
  rows = touched_rows(rp, eid, num_sc_per_device=num_sc_per_device,
                      num_scs=num_scs, table_rows=table.shape[0])
  hyper = [np.float32(np.asarray(h, np.float32).reshape(())) for h in
           hyperparameters]
  out = update_fn(sums[rows], table[rows], *[s[rows] for s in slots], *hyper)
  outs = list(out) if isinstance(out, (list, tuple)) else [out]
  new_table = np.asarray(outs[0], np.float32)
  if min_value is not None:
    new_table = np.maximum(new_table, np.float32(min_value))
  if max_value is not None:
    new_table = np.minimum(new_table, np.float32(max_value))
  table[rows] = new_table
  for s, v in zip(slots, outs[1:]):
    s[rows] = np.asarray(v, np.float32)
  return (table, *slots)
