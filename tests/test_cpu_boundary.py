"""CPU checks of the C-ABI boundary and the host-side API (no GPU needed)."""

import ctypes
import os
import re

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils as prim_utils
from oracle import refcpu

_HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include",
                       "scemb.h")


def _declared_functions():
  text = open(_HEADER).read()
  text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
  return sorted(set(re.findall(r"\b(scemb_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
  assert _declared_functions() == sorted(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
  lib = _native.load_library()
  for name in _declared_functions():
    assert hasattr(lib, name), name
  assert lib.scemb_version() >= 1
  assert lib.scemb_last_error() is not None


@pytest.mark.parametrize("max_ids,g,s", [(16, 1, 4), (1, 1, 1), (100, 2, 2),
                                         (1703936, 1, 1)])
def test_size_helpers_match_oracle(max_ids, g, s):
  lib = refcpu.lib()
  for mb in (False, True):
    assert pip.compute_theoretical_max_coo_buffer_size(
        max_ids, g, s, enable_minibatching=mb) == \
        lib.ref_theoretical_max_coo_buffer_size_ex(max_ids, g, s, int(mb))
    for suggested in (0, 48, 96, 1024, 10**6, 10**8):
      exp = lib.ref_coo_buffer_size_per_device_ex(max_ids, suggested, g, s,
                                                  int(mb))
      got = _native.load_library().scemb_compute_coo_buffer_size_per_device(
          max_ids, suggested, g, s, int(mb))
      assert got == exp
  assert pip.compute_row_pointers_size_per_device(g, s) == max(g * s, 8) * s
  # GetRowPointersSizePerDevice: 64 buckets with minibatching
  # (input_preprocessing_util.h:497-511).
  assert pip.compute_row_pointers_size_per_device(
      g, s, enable_minibatching=True) == max(g * s, 8) * s * 64


def test_size_helper_kats():
  """input_preprocessing_util_test.cc:99-133; pybind test :1992-2060."""
  assert pip.compute_theoretical_max_coo_buffer_size(16, 1, 4) == 256
  lib = _native.load_library()
  assert lib.scemb_compute_coo_buffer_size_per_device(16, 48, 1, 4, 0) == 64
  assert lib.scemb_compute_coo_buffer_size_per_device(16, 96, 1, 4, 0) == 96
  assert lib.scemb_compute_coo_buffer_size_per_device(16, 1024, 1, 4, 0) == -1
  assert lib.scemb_compute_coo_buffer_size_per_device(16, 1024, 1, 4, 1) == \
      1024
  assert pip.compute_row_pointers_size_per_device(1, 4) == 32
  assert pip.compute_row_pointers_size_per_device(4, 4) == 64


def test_primitive_validation_messages():
  """Abstract-eval checks of lib/core/primitives/utils.py:79-155."""
  rp = np.array([0, 1, 2, 4], np.int32)
  ids = np.array([0, 1, 2, 3], np.int32)
  gains = np.ones(4, np.float32)
  table = np.ones((2, 4), np.float32)
  grad = np.ones((2, 4), np.float32)
  ok = dict(max_ids_per_partition=16, max_unique_ids_per_partition=16,
            computation_name="c", sharding_strategy=1)
  prim_utils.validate_abstract_eval_params(rp, ids, ids, gains, 1, table,
                                           grad, **ok)
  with pytest.raises(ValueError, match="lhs_row_pointers must have type"):
    prim_utils.validate_abstract_eval_params(rp.astype(np.float32), ids, ids,
                                             gains, 1, table, grad, **ok)
  with pytest.raises(ValueError, match="lhs_gains must have type"):
    prim_utils.validate_abstract_eval_params(rp, ids, ids,
                                             gains.astype(np.int32), 1, table,
                                             grad, **ok)
  with pytest.raises(ValueError, match="embedding_table must have dim"):
    prim_utils.validate_abstract_eval_params(rp, ids, ids, gains, 1,
                                             np.ones((1, 2, 3), np.float32),
                                             grad, **ok)
  with pytest.raises(ValueError, match="equal rank 1 shapes"):
    prim_utils.validate_abstract_eval_params(rp, ids[:3], ids, gains, 1,
                                             table, grad, **ok)
  with pytest.raises(ValueError, match="equal feature"):
    prim_utils.validate_abstract_eval_params(rp, ids, ids, gains, 1, table,
                                             np.ones((2, 5), np.float32), **ok)
  with pytest.raises(ValueError, match="sharding_strategy must be MOD"):
    prim_utils.validate_abstract_eval_params(
        rp, ids, ids, gains, 1, table, grad,
        **{**ok, "sharding_strategy": 2})
  with pytest.raises(ValueError, match="max_ids_per_partition must be"):
    prim_utils.validate_abstract_eval_params(
        rp, ids, ids, gains, 1, table, grad,
        **{**ok, "max_ids_per_partition": 0})
  with pytest.raises(ValueError, match="computation_name"):
    prim_utils.validate_abstract_eval_params(
        rp, ids, ids, gains, 1, table, grad, **{**ok, "computation_name": ""})
  with pytest.raises(ValueError, match="min_value must be less"):
    prim_utils.validate_abstract_eval_params(rp, ids, ids, gains, 1, table,
                                             grad, **ok, min_value=2.0,
                                             max_value=1.0)


def _sizing_call(build_view, local_devices, table_rows=1024,
                 enable_minibatching=0, minibatching_pass=0, split=0,
                 flags=0, valency=2, allow_dropping=0):
  """scemb_preprocess_workspace_size for one 64 x `valency` dense feature
  (sizing only: no device memory is touched)."""
  lib = _native.load_library()
  feat = (_native.Feature * 1)()
  feat[0] = _native.Feature(None, None, None, None, 64, 64 * valency, valency,
                            0, 0, 0)
  opts = _native.PreprocessOptions(local_devices, local_devices, 1, 0, 512,
                                   512, allow_dropping, 0, 512, 1024,
                                   int(build_view), enable_minibatching,
                                   table_rows, minibatching_pass, flags, split)
  return int(lib.scemb_preprocess_workspace_size(feat, 1, ctypes.byref(opts)))


def test_grouping_route_selection():
  """The route that merges duplicates at extraction needs less workspace
  than the after-sort route; the flag, id dropping, minibatching and rows
  longer than 896 ids each select the after-sort route."""
  at_extraction = _sizing_call(False, 1)
  after_sort = _sizing_call(False, 1, flags=_native.PREPROCESS_GROUP_AFTER_SORT)
  assert 0 < at_extraction < after_sort
  assert _sizing_call(False, 1, allow_dropping=1) == after_sort
  assert _sizing_call(True, 1) < _sizing_call(
      True, 1, flags=_native.PREPROCESS_GROUP_AFTER_SORT)
  long_rows = _sizing_call(False, 1, valency=897)
  assert long_rows == _sizing_call(
      False, 1, valency=897, flags=_native.PREPROCESS_GROUP_AFTER_SORT)
  assert _sizing_call(False, 1, valency=896) < _sizing_call(
      False, 1, valency=896, flags=_native.PREPROCESS_GROUP_AFTER_SORT)


def test_check_row_splits():
  """One pass over host row splits: the longest row, or the reference's
  RaggedTensorInputBatch contract violated (start 0, non-decreasing, end at
  the number of values)."""
  lib = _native.load_library()

  def check(splits, nnz):
    a = np.ascontiguousarray(splits, dtype=np.int64)
    out = ctypes.c_int64(-1)
    rc = lib.scemb_check_row_splits(a.ctypes.data, a.size - 1, nnz,
                                    ctypes.byref(out))
    return rc, out.value

  assert check([0, 2, 2, 7, 8], 8) == (0, 5)
  assert check([0], 0) == (0, 0)
  assert check([0, 0, 0], 0) == (0, 0)
  assert check([1, 2, 3], 3)[0] == _native.SCEMB_ERR_INVALID_ARGUMENT
  assert check([0, 3, 2, 4], 4)[0] == _native.SCEMB_ERR_INVALID_ARGUMENT
  assert b"non-decreasing" in lib.scemb_last_error()
  assert check([0, 2, 4], 5)[0] == _native.SCEMB_ERR_INVALID_ARGUMENT
  assert pip._check_row_splits(np.array([0, 1, 4], np.int64), 4) == 3  # pylint: disable=protected-access
  with pytest.raises(ValueError, match="non-decreasing"):
    pip._check_row_splits(np.array([0, 4, 1], np.int64), 1)  # pylint: disable=protected-access
  with pytest.raises(ValueError, match="non-decreasing"):
    pip._check_row_splits(np.zeros(0, np.int64), 0)  # pylint: disable=protected-access


def test_stage_row_splits_copies_and_checks():
  """The staging variant copies the splits while it checks them."""
  lib = _native.load_library()
  rng = np.random.default_rng(0)
  for rows in (0, 1, 3, 4, 5, 1000, 16385):
    src = np.zeros(rows + 1, np.int64)
    src[1:] = np.cumsum(rng.integers(0, 9, size=rows))
    dst = np.full(rows + 1, -7, np.int64)
    out = ctypes.c_int64(-1)
    assert lib.scemb_stage_row_splits(src.ctypes.data, rows, int(src[-1]),
                                      dst.ctypes.data, ctypes.byref(out)) == 0
    np.testing.assert_array_equal(dst, src)
    assert out.value == (int(np.diff(src).max()) if rows else 0)
  bad = np.array([0, 5, 3, 6], np.int64)
  dst = np.zeros(4, np.int64)
  assert lib.scemb_stage_row_splits(bad.ctypes.data, 3, 6, dst.ctypes.data,
                                    ctypes.byref(out)) == \
      _native.SCEMB_ERR_INVALID_ARGUMENT


def _stage_batch(splits, nnz=None):
  """scemb_stage_row_splits_batch over `splits`: (rc, first_bad, copies,
  longest rows)."""
  lib = _native.load_library()
  n = len(splits)
  dsts = [np.full(s.size, -7, np.int64) for s in splits]
  src = np.array([s.ctypes.data for s in splits], np.uint64)
  dst = np.array([d.ctypes.data for d in dsts], np.uint64)
  rows = np.array([s.size - 1 for s in splits], np.int64)
  nnz = np.array([int(s[-1]) for s in splits] if nnz is None else nnz,
                 np.int64)
  longest = np.full(n, -1, np.int64)
  bad = ctypes.c_int32(-2)
  rc = lib.scemb_stage_row_splits_batch(n, src.ctypes.data, rows.ctypes.data,
                                        nnz.ctypes.data, dst.ctypes.data,
                                        longest.ctypes.data, ctypes.byref(bad))
  return rc, bad.value, dsts, longest


def test_stage_row_splits_batch_matches_one_at_a_time():
  """The batched staging copies and checks every feature as the one-feature
  call does, with features long enough to be split over threads (the
  longest row placed in a late chunk), and names the first bad feature."""
  rng = np.random.default_rng(1)
  sizes = (0, 1, 7, 1000, 16385, 32768, 32769, 200_003, 70_000, 3)
  splits = []
  for rows in sizes:
    s = np.zeros(rows + 1, np.int64)
    s[1:] = np.cumsum(rng.integers(0, 9, size=rows))
    if rows > 100_000:
      s[rows - 5:] += 1000  # the longest row, in the last chunk
    splits.append(s)
  rc, first_bad, dsts, longest = _stage_batch(splits)
  assert rc == 0 and first_bad == -1
  for s, d, most in zip(splits, dsts, longest.tolist()):
    np.testing.assert_array_equal(d, s)
    assert most == (int(np.diff(s).max()) if s.size > 1 else 0)
  assert longest[sizes.index(200_003)] >= 1000
  # A decrease inside a middle chunk of a long feature; a wrong end; a
  # non-zero start.
  dec = splits[7].copy()
  dec[100_000] = dec[99_999] - 1
  rc, first_bad, _, _ = _stage_batch([splits[3], dec, splits[8]])
  assert rc == _native.SCEMB_ERR_INVALID_ARGUMENT and first_bad == 1
  rc, first_bad, _, _ = _stage_batch(
      [splits[3], splits[4]], nnz=[int(splits[3][-1]), int(splits[4][-1]) + 1])
  assert rc == _native.SCEMB_ERR_INVALID_ARGUMENT and first_bad == 1
  start = splits[2].copy() + 1
  rc, first_bad, _, _ = _stage_batch([start])
  assert rc == _native.SCEMB_ERR_INVALID_ARGUMENT and first_bad == 0
  assert _stage_batch([])[0] == 0


def test_preprocess_minibatching_options():
  """The bucket passes size 64 buckets per (SC, partition); a bad pass or a
  split of 64 bits is refused; the sample view adds its temporaries."""
  plain = _sizing_call(False, 1, enable_minibatching=1)
  bucket = _sizing_call(False, 1, enable_minibatching=1, minibatching_pass=1)
  assert plain > 0 and bucket > plain
  assert _sizing_call(False, 1, enable_minibatching=1, minibatching_pass=2,
                      split=0b101) > 0
  assert _sizing_call(False, 1, enable_minibatching=1,
                      minibatching_pass=3) == 0
  assert b"minibatching_pass" in _native.load_library().scemb_last_error()
  assert _sizing_call(True, 1, enable_minibatching=1) > plain
  assert _sizing_call(False, 1, enable_minibatching=1, minibatching_pass=2,
                      split=1 << 63) == 0


def test_preprocess_sample_view_option():
  """build_sample_view adds the view temporaries to the workspace and is
  refused for several devices or a table that does not split into
  partitions (the options struct layout is read as the header declares)."""
  plain = _sizing_call(False, 1)
  with_view = _sizing_call(True, 1)
  assert plain > 0 and with_view > plain
  assert _sizing_call(True, 2) == 0
  assert b"one local and one global device" in \
      _native.load_library().scemb_last_error()
  assert _sizing_call(True, 1, table_rows=0) == 0
  assert _sizing_call(False, 2) > 0


def test_embedding_size_helpers_with_minibatching():
  """lib/nn/tests/embedding_test.py:964-1000."""
  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top
  kw = dict(max_ids_per_partition=12, global_device_count=1,
            num_sc_per_device=4)
  assert embedding.compute_theoretical_max_coo_buffer_size(
      **kw, enable_minibatching=False) == 256
  assert embedding.compute_theoretical_max_coo_buffer_size(
      **kw, enable_minibatching=True) == 16384
  assert embedding.compute_row_pointers_size_per_device(
      global_device_count=1, num_sc_per_device=4,
      enable_minibatching=False) == 32
  assert embedding.compute_row_pointers_size_per_device(
      global_device_count=1, num_sc_per_device=4,
      enable_minibatching=True) == 2048


def test_device_status_decoding():
  """Validation mode's status check names every bit the kernels set."""
  _native.raise_on_status(0, "op")
  with pytest.raises(RuntimeError, match=r"op: device status 0x8: .*repeats"):
    _native.raise_on_status(_native.STATUS_SHARED_ROW, "op")
  with pytest.raises(RuntimeError, match="out of range.*not valid"):
    _native.raise_on_status(
        _native.STATUS_BAD_ENTRY | _native.STATUS_UNSORTED, "op")
  prev = _native.set_validation(False)
  try:
    assert _native.status_word() is None
    _native.check_status_word(None, "op")
  finally:
    _native.set_validation(prev)


def test_unknown_row_length_is_not_one_id_per_row():
  """A ragged feature whose longest row is not known yet (row splits
  staged, not checked) is not declared one id per row; 0 and 1 known ids
  per row are; a dense feature follows its valency."""
  splits = np.array([0, 1, 3], np.int64)
  kw = dict(ids=None, weights=None, splits=None, splits_host=splits,
            num_rows=2, nnz=3, valency=0, max_id=None)
  assert not pip._DeviceFeature(**kw).one_id_per_row  # pylint: disable=protected-access
  assert not pip._DeviceFeature(**kw, max_row_length=2).one_id_per_row  # pylint: disable=protected-access
  assert pip._DeviceFeature(**kw, max_row_length=1).one_id_per_row  # pylint: disable=protected-access
  assert pip._DeviceFeature(**kw, max_row_length=0).one_id_per_row  # pylint: disable=protected-access
  kw.update(splits_host=None, valency=1)
  assert pip._DeviceFeature(**kw).one_id_per_row  # pylint: disable=protected-access
  kw.update(valency=3)
  assert not pip._DeviceFeature(**kw).one_id_per_row  # pylint: disable=protected-access
