"""Argument errors of the preprocessing, on the CPU (no device work starts).

Transcribed from the reference's status tests:
  lib/core/tests/pybind_input_preprocessing_test.py:1871-1990 (the Python
      entry raises ValueError with these messages), and
  lib/core/tests/input_preprocessing_test.cc:1321-1480 (the C++ entry
      returns InvalidArgument with the same messages).
Both layers are checked: the Python entry (pybind_input_preprocessing and
the embedding API), and the C ABI through ctypes, whose planner runs on the
host before anything is enqueued (scemb_preprocess_workspace_size returns 0
and scemb_last_error() holds the message).

Also here: the C ABI refuses weighted features whose sample rows do not
ascend across the stack when id dropping is on. The reference merges a
duplicate (row, column) into the last kept entry across a dropped one
(sort_and_group_coo_tensors_impl.h:251-259); this build merges adjacent
duplicates, which agrees whenever rows ascend, as they always do for
features in row_offset order (the only order the Python entry produces).
"""

import ctypes

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip
from jax_tpu_embedding.sparsecore.lib.nn import embedding
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec

SINGLETON = np.array([[5], [18], [0], [20], [6], [15], [12], [7], [3], [11],
                      [8], [26], [0], [18], [7], [2]], dtype=np.int32)
SINGLETON_WEIGHTS = np.ones((16, 1), np.float32)


def _singleton_spec():
  table = embedding_spec.TableSpec(
      vocabulary_size=16, embedding_dim=8, initializer=None,
      optimizer=embedding_spec.SGDOptimizerSpec(learning_rate=0.001),
      combiner="sum", name="singleton_features_table",
      max_ids_per_partition=12, max_unique_ids_per_partition=12)
  spec = embedding_spec.FeatureSpec(
      table_spec=table, input_shape=[16, 1], output_shape=[16, 8],
      name="singleton_input_feature")
  embedding.prepare_feature_specs_for_training([spec], 1, 4)
  return spec


# (local_device_count, global_device_count, num_sc_per_device, message)
CASES = [
    (0, 1, 4, "local_device_count must be greater than 0"),
    (1, 0, 4, "global_device_count must be greater than 0"),
    (2, 1, 4, "global_device_count must be greater than or equal to "
     "local_device_count"),
    (1, 1, 0, "num_sc_per_device must be greater than 0"),
    (1, 1, 3, "must be a power of 2"),
]


@pytest.mark.parametrize("local,glob,num_sc,msg", CASES)
def test_pybind_entry_raises(local, glob, num_sc, msg):
  with pytest.raises(ValueError, match=msg):
    pip.preprocess_sparse_dense_matmul_input(
        [SINGLETON], [SINGLETON_WEIGHTS], [_singleton_spec()], local, glob,
        num_sc_per_device=num_sc, batch_number=42)


def test_pybind_invalid_sharding_strategy_raises():
  with pytest.raises((ValueError, TypeError)):
    pip.preprocess_sparse_dense_matmul_input(
        [SINGLETON], [SINGLETON_WEIGHTS], [_singleton_spec()], 1, 1,
        num_sc_per_device=4, sharding_strategy=0, batch_number=42)


def test_pybind_empty_input_batches_raises():
  with pytest.raises(ValueError, match="input_batches cannot be empty"):
    pip.preprocess_sparse_dense_matmul_input([], [], [], 1, 1,
                                             num_sc_per_device=4,
                                             batch_number=42)


@pytest.mark.parametrize("local,glob,msg", [c[:2] + c[3:] for c in CASES[:3]])
def test_embedding_entry_raises(local, glob, msg):
  spec = _singleton_spec()
  with pytest.raises(ValueError, match=msg):
    embedding.preprocess_sparse_dense_matmul_input(
        [SINGLETON], None, [spec], local, glob, num_sc_per_device=4)


# --- the C ABI --------------------------------------------------------------


def _feature(num_rows, row_offset, weights=False):
  f = _native.Feature()
  f.ids = 0
  f.weights = 16 if weights else 0  # never read by the planner
  f.row_splits = 0
  f.row_splits_host = 0
  f.num_rows = num_rows
  f.nnz = num_rows
  f.valency = 1
  f.row_offset = row_offset
  f.col_offset = 0
  f.col_shift = 0
  return f


def _options(local=1, glob=1, num_sc=4, weights=False, dropping=False):
  o = _native.PreprocessOptions()
  o.local_device_count = local
  o.global_device_count = glob
  o.num_sc_per_device = num_sc
  o.combiner = 0
  o.max_ids_per_partition = 4
  o.max_unique_ids_per_partition = 4
  o.allow_id_dropping = int(dropping)
  o.has_variable_weights = int(weights)
  o.coo_buffer_size_per_device = 1024
  o.col_id_bound = 64
  return o


def _plan_error(features, options):
  lib = _native.load_library()
  arr = (_native.Feature * max(1, len(features)))(*features)
  size = lib.scemb_preprocess_workspace_size(arr, len(features),
                                             ctypes.byref(options))
  return size, lib.scemb_last_error().decode()


@pytest.mark.parametrize("local,glob,num_sc,msg", CASES)
def test_c_abi_returns_invalid_argument(local, glob, num_sc, msg):
  size, err = _plan_error([_feature(16, 0)], _options(local, glob, num_sc))
  assert size == 0
  assert msg in err


def test_c_abi_messages_carry_the_values():
  assert _plan_error([_feature(16, 0)], _options(0, 1, 4))[1] == (
      "local_device_count must be greater than 0, but got 0")
  assert _plan_error([_feature(16, 0)], _options(2, 1, 4))[1] == (
      "global_device_count must be greater than or equal to "
      "local_device_count, but got 1 vs 2")
  assert _plan_error([_feature(16, 0)], _options(1, 1, 3))[1] == (
      "Total number of SparseCores (3) must be a power of 2.")


def test_c_abi_empty_input_batches():
  size, err = _plan_error([], _options())
  assert size == 0
  assert err == "input_batches cannot be empty."


def test_c_abi_refuses_weighted_rows_out_of_order_with_dropping():
  # The second feature's samples come before the first one's.
  feats = [_feature(16, 16), _feature(16, 0)]
  size, err = _plan_error(feats, _options(weights=True, dropping=True))
  assert size == 0
  assert "row_offset order" in err
  # Unweighted, without dropping, or in order: the planner accepts it (and
  # sizes the workspace).
  for weights, dropping, order in ((False, True, (16, 0)),
                                   (True, False, (16, 0)),
                                   (True, True, (0, 16))):
    feats = [_feature(16, order[0]), _feature(16, order[1])]
    size, _ = _plan_error(feats, _options(weights=weights, dropping=dropping))
    assert size > 0
