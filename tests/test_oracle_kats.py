"""Pins the CPU oracle against the reference's own known-answer tests.

Every expected value below is transcribed from the reference test cited in the
test's docstring (paths relative to jax_tpu_embedding/sparsecore/). These run
on the CPU only; the GPU parity tests then compare libscemb.so to this oracle.
"""

import math

import numpy as np
import pytest

from oracle import refcpu

INT_MAX = 2**31 - 1


# --------------------------------------------------------------------------
# coo_format.h: column ids and grouping keys.
# --------------------------------------------------------------------------


def test_col_ids_kat():
  """lib/core/tests/input_preprocessing_util_test.cc:44-63."""
  assert refcpu.get_col_id(2, 4, 32, 3) == 34
  assert refcpu.get_col_id(38, 0, 0, 3) == 38
  assert refcpu.get_col_id(10, 0, 32, 7) == 42
  assert refcpu.get_col_id(26, 0, 0, 3) == 26
  # input_preprocessing_test.cc:548-562: 128%4 + 127//4*4 + 32 = 156.
  assert refcpu.get_col_id(127, 1, 32, 3) == 156
  assert refcpu.get_col_id(70, 0, 0, 3) == 70


def test_col_id_property():
  """GetColIdIsCorrect (input_preprocessing_util_test.cc:65-82), sampled."""
  rng = np.random.default_rng(0)
  for _ in range(3000):
    emb = int(rng.integers(0, 100_000_001))
    shift = int(rng.integers(0, 65))
    off_per_shard = int(rng.integers(0, 600_001))
    bits = int(rng.integers(0, 10))
    ns = 1 << bits
    col = refcpu.get_col_id(emb, shift, off_per_shard * ns, ns - 1)
    if col < 0:  # int32 overflow domain of the reference as well
      continue
    assert col % ns == (emb + shift) % ns
    assert col // ns == (emb + off_per_shard * ns) // ns


def test_grouping_key_layout():
  """coo_format.h:154-185 layout; input_preprocessing_test.cc:566-579."""
  # Bits [57:26] hold rotr32(col, log2 NS), bits [25:0] the data field.
  key = refcpu.grouping_key(0b1011, 5, 2)
  rot = (0b1011 >> 2) | ((0b1011 & 3) << 30)
  assert key == (rot << 26) | 5
  assert refcpu.col_id_from_key(key, 2) == 0b1011
  assert refcpu.data_from_key(key) == 5
  # Keys generated in (partition, local id, index) order sort ascending and
  # return their index (KeysAreSorted / IndexFromKeyIsCorrect).
  keys, index = [], 0
  for p in range(4):
    for local in range(3):
      keys.append(refcpu.grouping_key(local * 4 + p, index, 2))
      index += 1
  assert all(a < b for a, b in zip(keys, keys[1:]))
  assert [refcpu.data_from_key(k) for k in keys] == list(range(len(keys)))


# --------------------------------------------------------------------------
# Extraction: ragged_tensor_input_batch_test.cc and input_preprocessing_test.cc
# --------------------------------------------------------------------------


def _ragged_abc():
  # Input: (0,0), (0,1), (0,2), (1,0), (2,0), (3,2)
  return refcpu.RaggedFeature(np.array([0, 1, 2, 0, 0, 2]),
                              np.array([0, 3, 4, 5, 6]))


def _coo(rows, cols, gains):
  return list(zip(rows.tolist(), cols.tolist(), gains.tolist()))


def test_ragged_slice_sum():
  """ragged_tensor_input_batch_test.cc:32-98."""
  f = _ragged_abc()
  r = refcpu.extract_slice(f, 0, 4, 0, 0, 0, 4, "sum")
  assert _coo(*r) == [(0, 0, 1.0), (0, 1, 1.0), (0, 2, 1.0), (1, 0, 1.0),
                      (2, 0, 1.0), (3, 2, 1.0)]
  r = refcpu.extract_slice(f, 1, 3, 0, 0, 0, 4, "sum")
  assert _coo(*r) == [(0, 0, 1.0), (1, 0, 1.0)]
  r = refcpu.extract_slice(f, 2, 4, 16, 8, 0, 4, "sum")
  assert _coo(*r) == [(16, 8, 1.0), (17, 10, 1.0)]


def test_ragged_slice_mean():
  """ragged_tensor_input_batch_test.cc:100-121."""
  r = refcpu.extract_slice(_ragged_abc(), 0, 4, 0, 0, 0, 4, "mean")
  third = np.float32(1.0) / np.float32(3)
  assert _coo(*r) == [(0, 0, third), (0, 1, third), (0, 2, third),
                      (1, 0, 1.0), (2, 0, 1.0), (3, 2, 1.0)]


def test_ragged_slice_sqrtn():
  """ragged_tensor_input_batch_test.cc:123-139."""
  r = refcpu.extract_slice(_ragged_abc(), 0, 4, 0, 0, 0, 4, "sqrtn")
  g = np.float32(1.0) / np.sqrt(np.float32(3))
  assert _coo(*r) == [(0, 0, g), (0, 1, g), (0, 2, g), (1, 0, 1.0),
                      (2, 0, 1.0), (3, 2, 1.0)]
  assert abs(r[2][0] - 1.0 / math.sqrt(3)) < 1e-7


_INPUT_A = ([5, 18, 18, 0, 0, 20, 18, 0, 18, 0, 0, 20, 5, 18, 18, 0],
            [0, 2, 4, 6, 8, 10, 12, 14, 16])
_INPUT_B = ([2, 10, 1, 9, 3, 7, 4, 8], list(range(9)))
_INPUT_C = (sum([[i] * i for i in range(1, 9)], []),
            [0, 1, 3, 6, 10, 15, 21, 28, 36])
_INPUT_D = (sum([[i] * i for i in range(9, 17)], []),
            [0, 9, 19, 30, 42, 55, 69, 84, 100])


def test_extract_multi_process_split_then_stack():
  """input_preprocessing_test.cc:86-157 inputs, :226-290 expectations."""
  fa = refcpu.RaggedFeature(np.array(_INPUT_A[0]), np.array(_INPUT_A[1]),
                            row_offset=0, col_offset=0, col_shift=0)
  fb = refcpu.RaggedFeature(np.array(_INPUT_B[0]), np.array(_INPUT_B[1]),
                            row_offset=16, col_offset=32, col_shift=0)
  rows, cols, gains, sizes, bfd = refcpu.extract_device(
      [fa, fb], local_device_id=0, local_device_count=1,
      global_device_count=2, num_sc_per_device=4)
  assert bfd == 16
  assert len(rows) == 24
  expected = [
      (0, 5), (0, 18), (1, 18), (1, 0), (2, 34), (3, 42),
      (4, 0), (4, 20), (5, 18), (5, 0), (6, 33), (7, 41),
      (8, 18), (8, 0), (9, 0), (9, 20), (10, 35), (11, 39),
      (12, 5), (12, 18), (13, 18), (13, 0), (14, 36), (15, 40),
  ]
  assert list(zip(rows.tolist(), cols.tolist())) == expected
  assert np.all(gains == 1.0)
  assert sizes.tolist() == [6, 6, 6, 6]


def test_extract_single_process_sizes():
  """input_preprocessing_test.cc:292-318 (SingleProcessSingleDevice)."""
  fc = refcpu.RaggedFeature(np.array(_INPUT_C[0]), np.array(_INPUT_C[1]),
                            row_offset=0, col_offset=0)
  fd = refcpu.RaggedFeature(np.array(_INPUT_D[0]), np.array(_INPUT_D[1]),
                            row_offset=8, col_offset=32)
  rows, _, _, sizes, bfd = refcpu.extract_device(
      [fc, fd], local_device_id=0, local_device_count=1,
      global_device_count=1, num_sc_per_device=4)
  assert bfd == 16
  assert len(rows) == 16 * 17 // 2
  assert sizes.tolist() == [1 + 2 + 9 + 10, 3 + 4 + 11 + 12, 5 + 6 + 13 + 14,
                            7 + 8 + 15 + 16]


def test_extract_multi_chip_sizes():
  """input_preprocessing_test.cc:320-345 (MultiChipSplitThenStack)."""
  fc = refcpu.RaggedFeature(np.array(_INPUT_C[0]), np.array(_INPUT_C[1]),
                            row_offset=0, col_offset=0)
  fd = refcpu.RaggedFeature(np.array(_INPUT_D[0]), np.array(_INPUT_D[1]),
                            row_offset=8, col_offset=32)
  expected = [[1 + 9, 2 + 10, 3 + 11, 4 + 12], [5 + 13, 6 + 14, 7 + 15, 8 + 16]]
  for d in range(2):
    _, _, _, sizes, bfd = refcpu.extract_device(
        [fc, fd], local_device_id=d, local_device_count=2,
        global_device_count=2, num_sc_per_device=4)
    assert bfd == 8
    assert sizes.tolist() == expected[d]


# --------------------------------------------------------------------------
# Sort / group / dedupe / drop: input_preprocessing_util_test.cc
# --------------------------------------------------------------------------


def _test_extracted(num_sc, batch, coos):
  """ExtractedCooTensors test constructor (input_preprocessing_util.h:284-329)."""
  bps = batch // num_sc
  per = [[] for _ in range(num_sc)]
  for r, c, g in coos:
    per[r // bps].append((r, c, g))
  rows = np.array([x[0] for p in per for x in p], np.int32)
  cols = np.array([x[1] for p in per for x in p], np.int32)
  gains = np.array([x[2] for p in per for x in p], np.float32)
  sizes = np.array([len(p) for p in per], np.int64)
  return rows, cols, gains, sizes


def _group(num_sc, batch, coos, *, max_ids, max_unique, drop=False,
           num_scs=None):
  rows, cols, gains, sizes = _test_extracted(num_sc, batch, coos)
  return refcpu.sort_and_group(
      rows, cols, gains, sizes, num_scs=num_scs or num_sc,
      max_ids_per_partition=max_ids, max_unique_ids_per_partition=max_unique,
      allow_id_dropping=drop)


def _grouped(res, s):
  r, c, g = res.per_sc[s]
  return list(zip(r.tolist(), c.tolist(), g.tolist()))


def _rows_x_ids(nrows, ids):
  return [(row, i, 1.0) for row in range(nrows) for i in ids]


def test_sort_and_group_base():
  """SortAndGroupTest.Base (input_preprocessing_util_test.cc:135-215)."""
  res = _group(4, 8, _rows_x_ids(8, range(4)), max_ids=32, max_unique=32)
  for s in range(4):
    exp = [(2 * s + k, c, 1.0) for c in range(4) for k in range(2)]
    assert _grouped(res, s) == exp
  assert res.dropped_id_count == 0
  assert res.max_ids_per_partition.tolist() == [2, 2, 2, 2]
  assert res.max_unique_ids_per_partition.tolist() == [1, 1, 1, 1]
  assert res.required_buffer_size.tolist() == [32, 32, 32, 32]


def test_sort_and_group_two_scs():
  """SortAndGroupTest.TwoScs (input_preprocessing_util_test.cc:217-278)."""
  res = _group(2, 8, _rows_x_ids(8, range(4)), max_ids=32, max_unique=32)
  for s in range(2):
    exp = [(4 * s + k, c, 1.0) for c in (0, 2, 1, 3) for k in range(4)]
    assert _grouped(res, s) == exp
  assert res.dropped_id_count == 0
  assert res.max_ids_per_partition.tolist() == [8, 8]
  assert res.max_unique_ids_per_partition.tolist() == [2, 2]
  assert res.required_buffer_size.tolist() == [16, 16]


@pytest.mark.parametrize(
    "nrows,ids,max_ids,max_unique,exp_ids,exp_unique,exp_req",
    [
        # VerifyIdLimitations1..6 (input_preprocessing_util_test.cc:280-592).
        (8, range(4), 2, 1, [2] * 4, [1] * 4, [32] * 4),
        (16, range(4), 4, 1, [4] * 4, [1] * 4, [32] * 4),
        (16, range(8), 8, 2, [8] * 4, [2] * 4, [32] * 4),
        (128, range(8), 64, 2, [64] * 4, [2] * 4, [256] * 4),
        (128, (0, 4, 8, 16), 128, 4, [128, 0, 0, 0], [4, 0, 0, 0],
         [128] * 4),
    ])
def test_verify_id_limitations(nrows, ids, max_ids, max_unique, exp_ids,
                               exp_unique, exp_req):
  res = _group(4, nrows, _rows_x_ids(nrows, ids), max_ids=max_ids,
               max_unique=max_unique)
  assert not res.limit_exceeded
  assert res.dropped_id_count == 0
  assert res.max_ids_per_partition.tolist() == exp_ids
  assert res.max_unique_ids_per_partition.tolist() == exp_unique
  assert res.required_buffer_size.tolist() == exp_req


def test_verify_id_limitations6():
  """VerifyIdLimitations6 (input_preprocessing_util_test.cc:545-591)."""
  coos = [(row, row * 4, 1.0) for row in range(128)]
  res = _group(4, 128, coos, max_ids=32, max_unique=32)
  assert res.dropped_id_count == 0
  assert res.max_ids_per_partition.tolist() == [32, 0, 0, 0]
  assert res.max_unique_ids_per_partition.tolist() == [32, 0, 0, 0]
  assert res.required_buffer_size.tolist() == [32, 32, 32, 32]


def test_id_dropping():
  """SortAndGroupTest.IdDropping (input_preprocessing_util_test.cc:593-693)."""
  res = _group(4, 16, _rows_x_ids(16, range(4)), max_ids=2, max_unique=1,
               drop=True)
  assert res.dropped_id_count == 32
  assert res.max_ids_per_partition.tolist() == [4, 4, 4, 4]
  assert res.max_unique_ids_per_partition.tolist() == [1, 1, 1, 1]
  assert res.required_buffer_size.tolist() == [32, 32, 32, 32]
  for s in range(4):
    exp = [(4 * s + k, c, 1.0) for c in range(4) for k in range(2)]
    assert _grouped(res, s) == exp


def test_limit_exceeded_without_dropping_is_fatal():
  """ValidateMaxIdsOrDie (sort_and_group_coo_tensors_impl.h:45-89)."""
  res = _group(4, 16, _rows_x_ids(16, range(4)), max_ids=2, max_unique=1)
  assert res.limit_exceeded


def test_dedupe_merges_gains_in_sorted_order():
  """Duplicates of (row, col) merge into the last kept entry.

  partitioned_coo_tensors.h:94-113; the Python reference's dedupe test
  (lib/core/tests/input_preprocessing_test.py:694-733) sums gains 1 + 2 = 3.
  """
  coos = [(0, 5, 1.0), (0, 5, 2.0), (0, 3, 0.25), (0, 5, 4.0), (1, 5, 0.5)]
  res = _group(1, 2, coos, max_ids=8, max_unique=8)
  assert _grouped(res, 0) == [(0, 3, 0.25), (0, 5, 7.0), (1, 5, 0.5)]
  assert res.max_ids_per_partition.tolist() == [3]
  assert res.max_unique_ids_per_partition.tolist() == [2]
  # With variable weights the key's data field is the extraction index, so
  # only runs adjacent after sorting merge (coo_format.h:154-185): a repeat
  # of (0, 5) after (1, 5) in extraction order stays a separate entry.
  coos = [(0, 5, 1.0), (1, 5, 0.5), (0, 5, 2.0)]
  res = _group(1, 2, coos, max_ids=8, max_unique=8)
  assert _grouped(res, 0) == [(0, 5, 1.0), (1, 5, 0.5), (0, 5, 2.0)]
  assert res.max_ids_per_partition.tolist() == [3]


# --------------------------------------------------------------------------
# CSR fill: input_preprocessing_util_test.cc:695-822
# --------------------------------------------------------------------------


def test_fill_buffer():
  """InputPreprocessingUtilTest.FillBuffer."""
  res = _group(4, 8, _rows_x_ids(8, range(4)), max_ids=32, max_unique=32)
  rp, eid, sid, gains, dropped = refcpu.fill_device(
      res.per_sc, num_scs=4, batch_size_per_sc=2, coo_size=160, rp_per_sc=8)
  assert rp.tolist() == [2, 10, 18, 26, 32, 32, 32, 32] * 4
  assert dropped == 0
  block_e = [0, 0] + [INT_MAX] * 6
  block_s = [0, 1] + [INT_MAX] * 6
  for s in range(4):
    seg = slice(40 * s, 40 * s + 32)
    assert eid[seg].tolist() == block_e * 4
    assert sid[seg].tolist() == block_s * 4
    g = gains[seg].reshape(4, 8)
    assert np.all(g[:, :2] == 1.0) and np.all(np.isnan(g[:, 2:]))
    # Positions 32..39 of each segment are left unwritten (`_`).
    assert eid[40 * s + 32:40 * s + 40].tolist() == [-7] * 8


def test_fill_buffer_static_overflow_drops():
  """A buffer smaller than required drops the tail (:74-95, :183-188)."""
  res = _group(1, 4, _rows_x_ids(4, range(4)), max_ids=32, max_unique=32)
  # 4 partitions x 4 ids would need 32 slots; give the segment 16.
  rp, eid, _, _, dropped = refcpu.fill_device(
      res.per_sc, num_scs=4, batch_size_per_sc=4, coo_size=16, rp_per_sc=8)
  assert dropped == 8
  assert rp.tolist() == [4, 12, 16, 16, 16, 16, 16, 16]
  assert eid[:4].tolist() == [0, 0, 0, 0]
  assert eid[4:8].tolist() == [INT_MAX] * 4


# --------------------------------------------------------------------------
# Buffer sizes: input_preprocessing_util_test.cc:99-133
# --------------------------------------------------------------------------


def test_coo_buffer_size():
  lib = refcpu.lib()
  assert lib.ref_coo_buffer_size_per_device(16, 0, 1, 4) == 16 * 4 * 4
  assert lib.ref_coo_buffer_size_per_device(16, 48, 1, 4) == 64
  assert lib.ref_coo_buffer_size_per_device(16, 96, 1, 4) == 96
  assert lib.ref_coo_buffer_size_per_device(16, 1024, 1, 4) == -1


# --------------------------------------------------------------------------
# Weighted gains (process_coo_tensors_impl.h:54-74, :118): mean uses a float
# running sum, sqrtn sums double squares into a float accumulator.
# --------------------------------------------------------------------------


def test_weighted_mean_and_sqrtn_gains():
  w = np.array([0.1, 0.7, 0.3, 2.5, 1e-3], np.float32)
  f = refcpu.RaggedFeature(np.arange(5), np.array([0, 5]), w)
  _, _, g = refcpu.extract_slice(f, 0, 1, 0, 0, 0, 1, "mean")
  s = np.float32(0)
  for x in w:
    s = np.float32(s + x)
  assert g.tolist() == (w / s).tolist()
  _, _, g = refcpu.extract_slice(f, 0, 1, 0, 0, 0, 1, "sqrtn")
  acc = np.float32(0)
  for x in w:
    acc = np.float32(np.float64(acc) + np.float64(x) * np.float64(x))
  assert g.tolist() == (w / np.sqrt(acc)).tolist()
  # Closed form check: a constant row of k weights w gives 1/sqrt(k).
  f2 = refcpu.RaggedFeature(np.arange(4), np.array([0, 4]),
                            np.full(4, 3.0, np.float32))
  _, _, g = refcpu.extract_slice(f2, 0, 1, 0, 0, 0, 1, "sqrtn")
  np.testing.assert_allclose(g, 0.5, rtol=0, atol=0)
  _, _, g = refcpu.extract_slice(f2, 0, 1, 0, 0, 0, 1, "mean")
  np.testing.assert_allclose(g, 0.25, rtol=0, atol=0)
