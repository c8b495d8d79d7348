"""The oracle's minibatching pieces against the reference's own tests and the
HighwayHash project's published vectors (CPU only).

* HighwayHash-64 (third-party google/highwayhash, which the reference calls
  through HighwayHashCatT, coo_format.h:43-49): the project's published
  64-bit test vectors (highwayhash_test.cc, key 0x0706050403020100 ...
  0x1F1E1D1C1B1A1918, input bytes 0, 1, 2, ..., sizes 0 to 64). They cover
  the 4-byte input the reference hashes, the remainder paths (sizes 1-31 mod
  32) and whole packets.
* ComputeMinibatchingSplit and MergeBuckets: minibatching_splits_test.cc:
  39-106 and the worked example of minibatching_splits_impl.h:33-50.
* PartitionedCooTensors::Merge: partitioned_coo_tensors_test.cc:114-221.
* Whole passes: MinibatchingCountTest (input_preprocessing_test.cc:587-725),
  the single-host cases of lib/nn/tests/minibatching_test.py:192-303, and
  properties that hold for any split (the minibatched CSR holds exactly the
  entries of the CSR without minibatching when nothing is dropped; the
  lookup over it gives the same activations).
"""

import types

import numpy as np
import pytest

from oracle import refcpu

HH_TEST_KEY = [0x0706050403020100, 0x0F0E0D0C0B0A0908, 0x1716151413121110,
               0x1F1E1D1C1B1A1918]
HH_EXPECTED64 = [
    0x907A56DE22C26E53, 0x7EAB43AAC7CDDD78, 0xB8D0569AB0B53D62,
    0x5C6BEFAB8A463D80, 0xF205A46893007EDA, 0x2B8A1668E4A94541,
    0xBD4CCC325BEFCA6F, 0x4D02AE1738F59482, 0xE1205108E55F3171,
    0x32D2644EC77A1584, 0xF6E10ACDB103A90B, 0xC3BBF4615B415C15,
    0x243CC2040063FA9C, 0xA89A58CE65E641FF, 0x24B031A348455A23,
    0x40793F86A449F33B, 0xCFAB3489F97EB832, 0x19FE67D2C8C5C0E2,
    0x04DD90A69C565CC2, 0x75D9518E2371C504, 0x38AD9B1141D3DD16,
    0x0264432CCD8A70E0, 0xA9DB5A6288683390, 0xD7B05492003F028C,
    0x205F615AEA59E51E, 0xEEE0C89621052884, 0x1BFC1A93A7284F4F,
    0x512175B5B70DA91D, 0xF71F8976A0A2C639, 0xAE093FEF1F84E3E7,
    0x22CA92B01161860F, 0x9FC7007CCF035A68, 0xA0C964D9ECD580FC,
    0x2C90F73CA03181FC, 0x185CF84E5691EB9E, 0x4FC1F5EF2752AA9B,
    0xF5B7391A5E0A33EB, 0xB9B84B83B4E96C9C, 0x5E42FE712A5CD9B4,
    0xA150F2F90C3F97DC, 0x7FA522D75E2D637D, 0x181AD0CC0DFFD32B,
    0x3889ED981E854028, 0xFB4297E8C586EE2D, 0x6D064A45BB28059C,
    0x90563609B3EC860C, 0x7AA4FCE94097C666, 0x1326BAC06B911E08,
    0xB926168D2B154F34, 0x9919848945B1948D, 0xA2A98FC534825EBE,
    0xE9809095213EF0B6, 0x582E5483707BC0E9, 0x086E9414A88A6AF5,
    0xEE86B98D20F6743D, 0xF89B7FF609B1C0A7, 0x4C7D9CC19E22C3E8,
    0x9A97005024562A6F, 0x5DD41CF423E6EBEF, 0xDF13609C0468E227,
    0x6E0DA4F64188155A, 0xB755BA4B50D7D4A1, 0x887A3484647479BD,
    0xAB8EEBE9BF2139A0, 0x75542C5D4CD2A6FF,
]
# coo_format.h:31-36
BUCKET_KEY = [0x4451e30f87db9609, 0xca7358a1fd2737f8, 0x4b2c991fcee4fdea,
              0x0b2658e18326f6ba]


@pytest.mark.parametrize("size", range(65))
def test_highway_hash_published_vectors(size):
  data = bytes(range(size))
  assert refcpu.highway_hash64(data, HH_TEST_KEY) == HH_EXPECTED64[size]


@pytest.mark.parametrize("col_id", [70, 156, 0, 1, 2**31 - 1, 123456789])
def test_bucket_is_highway_hash_of_the_int_column_id(col_id):
  """CooFormatTest.BucketIdCalculationIsCorrect (input_preprocessing_test.cc:
  546-562): bucket = HighwayHash(col_id) % 64 over the int's 4 bytes."""
  data = int(col_id).to_bytes(4, "little", signed=True)
  assert refcpu.minibatching_bucket(col_id) == \
      refcpu.highway_hash64(data, BUCKET_KEY) % 64


def test_buckets_spread_over_all_64():
  b = np.array([refcpu.minibatching_bucket(c) for c in range(4096)])
  counts = np.bincount(b, minlength=64)
  assert counts.min() > 30 and counts.max() < 100


SPLIT_CASES = [
    # minibatching_splits_test.cc:44-60
    ([10] * 8, 100, 0),
    ([100] * 8, 150, 0b1111111),
    ([10, 20, 30, 40, 50, 60, 70, 80], 100, 0b1101100),
    ([50, 50, 20, 80, 10, 10, 70, 10], 100, 0b1010000),
    ([90, 10, 90, 10, 90, 10, 90, 10], 100, 0b1110000),
    # minibatching_splits_impl.h:33-50
    ([2, 5, 1, 6, 3, 4, 2, 0], 7, 0b1110000),
]


@pytest.mark.parametrize("values,limit,expected", SPLIT_CASES)
def test_compute_minibatching_split(values, limit, expected):
  split, _ = refcpu.compute_minibatching_split(values, limit)
  assert split == expected


def test_compute_split_combines_counts_into_left_siblings():
  """minibatching_splits_impl.h:33-50: level by level the left sibling
  keeps the sum (no split) or the larger child (split)."""
  _, v = refcpu.compute_minibatching_split([2, 5, 1, 6, 3, 4, 2, 0], 7)
  # Level 1: 7, 7, 7, 2; level 2: split -> 7, split -> 7; level 3: split.
  assert v[0] == 7 and v[2] == 7 and v[4] == 7 and v[6] == 2


MERGE_CASES = [
    # minibatching_splits_test.cc:79-99 (unordered)
    (0b1111111, []),
    (0b0101101, [(2, 3), (0, 2), (0, 4)]),
    (0b0, [(0, 1), (2, 3), (4, 5), (6, 7), (0, 2), (4, 6), (0, 4)]),
    (0b0001010, [(0, 1), (4, 5), (0, 2), (4, 6), (0, 4)]),
    (0b0101010, [(0, 1), (4, 5), (0, 2), (0, 4)]),
]


@pytest.mark.parametrize("split,expected", MERGE_CASES)
def test_merge_buckets(split, expected):
  assert sorted(refcpu.merge_buckets(split, 8)) == sorted(expected)


def _coo(i):
  return (i, i, float(i))  # CooFormat(row i, col i, gain i)


def test_merge_all_two_buckets():
  """partitioned_coo_tensors_test.cc:114-146 (DevicePartitionedCooTensors
  MergeBuckets, two SCs, global_sc_count 2)."""
  sc0 = refcpu.merge_partitioned([[_coo(1)], [_coo(2)]], 2, 0)
  sc1 = refcpu.merge_partitioned([[_coo(3), _coo(4)], [_coo(5)]], 2, 0)
  assert sc0 == [[_coo(2), _coo(1)]]
  assert sc1 == [[_coo(3), _coo(4), _coo(5)]]


def test_partial_merge():
  """partitioned_coo_tensors_test.cc:148-186: split {2,3} -> minibatches
  {0,1,2} and {3}."""
  sc0 = refcpu.merge_partitioned([[_coo(1)], [_coo(2)], [_coo(3)], [_coo(4)]],
                                 2, 0b010)
  sc1 = refcpu.merge_partitioned([[_coo(5)], [_coo(6)], [_coo(7)], [_coo(8)]],
                                 2, 0b010)
  assert sc0 == [[_coo(2), _coo(1), _coo(3)], [_coo(4)]]
  assert sc1 == [[_coo(6), _coo(5), _coo(7)], [_coo(8)]]


def test_no_merge():
  """partitioned_coo_tensors_test.cc:188-221."""
  sc0 = refcpu.merge_partitioned([[_coo(1)], [_coo(2)], [_coo(3)], [_coo(4)]],
                                 2, 0b111)
  assert sc0 == [[_coo(1)], [_coo(2)], [_coo(3)], [_coo(4)]]


def minibatch_of_buckets(split, n=64):
  """Minibatch of each bucket from the merge tree: the boundary between
  buckets b - 1 and b belongs to the tree node whose subtree halves meet
  there; it separates two minibatches iff that node is split."""
  out, mb = [0], 0
  levels = n.bit_length() - 1
  for b in range(1, n):
    t = (b & -b).bit_length()  # level of the node (subtree size 2**t)
    index = sum(n >> l for l in range(1, t)) + (b >> t)
    assert t <= levels
    mb += (split >> index) & 1
    out.append(mb)
  return out


@pytest.mark.parametrize("seed", range(20))
def test_boundary_form_of_the_merge_tree(seed):
  """One entry per bucket: the minibatches that Merge forms are the runs
  of buckets between split boundaries (the closed form the GPU uses)."""
  rng = np.random.default_rng(seed)
  split = int(rng.integers(0, 2**63)) & int(rng.integers(0, 2**63))
  if seed == 0:
    split = 0
  if seed == 1:
    split = (1 << 63) - 1
  buckets = [[(b, 0, 1.0)] for b in range(64)]
  mbs = refcpu.merge_partitioned(buckets, 1, split)
  got = [0] * 64
  for m, entries in enumerate(mbs):
    for row, _, _ in entries:
      got[row] = m
  assert got == minibatch_of_buckets(split)
  assert len(mbs) == bin(split).count("1") + 1


# ---------------------------------------------------------------------------
# Whole passes.
# ---------------------------------------------------------------------------


def spec(name, stack, *, max_ids, max_unique, row_offset=0, col_offset=0,
         col_shift=0, batch=16, vocab=2048, combiner="sum", buffer=None):
  """A feature spec with the attributes preprocessing reads."""
  stacked = types.SimpleNamespace(
      max_ids_per_partition=max_ids, max_unique_ids_per_partition=max_unique,
      suggested_coo_buffer_size_per_device=buffer, combiner=combiner,
      stack_vocab_size=vocab)
  table = types.SimpleNamespace(
      name=name, vocabulary_size=vocab, stacked_table_spec=stacked,
      setting_in_stack=types.SimpleNamespace(stack_name=stack))
  return types.SimpleNamespace(
      name=name, table_spec=table, input_shape=[batch, 1],
      _id_transformation=types.SimpleNamespace(
          row_offset=row_offset, col_offset=col_offset, col_shift=col_shift))


def count_test_inputs(max_ids, max_unique, global_sc_count=4,
                      local_sc_count=4, batch=16):
  """CreateInputBatches of MinibatchingCountTest
  (input_preprocessing_test.cc:611-654): per SC, max_ids - max_unique ids
  i * global_sc_count, then max_unique ids 0.. max_unique - 1, spread over
  the SC's rows."""
  bps = batch // local_sc_count
  out = []
  for mi, mu in zip(max_ids, max_unique):
    ids = []
    for _ in range(local_sc_count):
      ids += [i * global_sc_count for i in range(mi - mu)]
      ids += list(range(mu))
    per_sc = len(ids) // local_sc_count
    per_row = per_sc // bps
    splits = [0]
    cur = 0
    for s in range(local_sc_count):
      for _ in range(bps - 1):
        cur += per_row
        splits.append(cur)
      cur = (s + 1) * per_sc
      splits.append(cur)
    rows = np.empty(batch, dtype=object)
    for r in range(batch):
      rows[r] = np.array(ids[splits[r]:splits[r + 1]], np.int32)
    out.append(rows)
  return out


def count_test_specs(limits):
  (i0, u0), (i1, u1) = limits
  return [spec("table_0", "table_0", max_ids=i0, max_unique=u0),
          spec("table_1", "table_0", max_ids=i1, max_unique=u1,
               row_offset=16, col_offset=32)]


def test_minibatch_count_when_not_required():
  """MinibatchingCountTest.SingleHostMinibatchCountIsCorrectWhenNotRequired
  (input_preprocessing_test.cc:666-691)."""
  feats = count_test_inputs([4, 6], [4, 6])
  res = refcpu.preprocess(feats, None, count_test_specs([(16, 16), (16, 16)]),
                          1, 1, num_sc_per_device=4, enable_minibatching=True)
  assert res.num_minibatches == 1


def test_minibatch_count_when_required():
  """...WhenRequired (input_preprocessing_test.cc:693-725): the stack's
  limits come from its first feature (5 ids, 2 unique)."""
  feats = count_test_inputs([10, 20], [5, 10])
  res = refcpu.preprocess(feats, None, count_test_specs([(5, 2), (5, 6)]),
                          1, 1, num_sc_per_device=4, enable_minibatching=True,
                          allow_id_dropping=True)
  assert res.num_minibatches > 1


def _random_rows(rng, batch, vocab, max_len):
  rows = np.empty(batch, dtype=object)
  for i in range(batch):
    rows[i] = rng.randint(0, vocab, size=(rng.randint(1, max_len + 1),),
                          dtype=np.int32)
  return rows


def _entries(rp, eid, sid, gains, S, ns, num_minibatches, batch, vocab):
  """(activation row, table row, gain) of every CSR entry, sorted."""
  out = []
  rp = np.asarray(rp).reshape(-1)
  if num_minibatches:
    rpb = len(rp) // (S * 64)
    prev = 0
    for s in range(S):
      for m in range(num_minibatches):
        for p in range(ns):
          start = -(-prev // 8) * 8
          end = int(rp[(s * num_minibatches + m) * rpb + p])
          for j in range(start, end):
            out.append((s * (batch // S) + int(sid[j]),
                        p * (vocab // ns) + int(eid[j]),
                        float(gains[j])))
          prev = max(end, start)
  else:
    rpb = len(rp) // S
    per = len(eid) // S
    for s in range(S):
      start = 0
      for p in range(ns):
        end = int(rp[s * rpb + p])
        for j in range(start, end):
          out.append((s * (batch // S) + int(sid[s * per + j]),
                      p * (vocab // ns) + int(eid[s * per + j]),
                      float(gains[s * per + j])))
        start = -(-end // 8) * 8
  return sorted(out)


@pytest.mark.parametrize("seed,S,limit", [(0, 1, 5), (1, 4, 2), (2, 2, 4),
                                          (3, 4, 2), (4, 1, 1000)])
def test_minibatched_csr_holds_the_same_entries(seed, S, limit):
  """Without drops, the minibatched CSR holds exactly the entries of the
  CSR without minibatching, and the lookup over it (the oracle, reading
  the minibatching layout) gives the same activations."""
  rng = np.random.RandomState(seed)
  batch, vocab = 32, 512
  feats = [_random_rows(rng, batch, vocab, 6)]
  specs = [spec("t", "t", max_ids=limit, max_unique=limit, batch=batch,
                vocab=vocab)]
  big = [spec("t", "t", max_ids=4096, max_unique=4096, batch=batch,
              vocab=vocab)]
  mb = refcpu.preprocess(feats, None, specs, 1, 1, num_sc_per_device=S,
                         enable_minibatching=True, allow_id_dropping=True)
  assert mb.dropped_id_count["t"] == 0
  ref = refcpu.preprocess(feats, None, big, 1, 1, num_sc_per_device=S)
  assert (mb.num_minibatches > 1) == (limit < 1000)
  got = _entries(mb.row_pointers["t"], mb.embedding_ids["t"],
                 mb.sample_ids["t"], mb.gains["t"], S, S,
                 mb.num_minibatches, batch, vocab)
  exp = _entries(ref.row_pointers["t"], ref.embedding_ids["t"],
                 ref.sample_ids["t"], ref.gains["t"], S, S, 0, batch, vocab)
  assert got == exp
  table = np.arange(vocab, dtype=np.float32)[:, None] * np.ones(
      (1, 4), np.float32)
  a = refcpu.sparse_dense_matmul(mb.row_pointers["t"], mb.embedding_ids["t"],
                                 mb.sample_ids["t"], mb.gains["t"], table,
                                 batch, num_sc_per_device=S, num_scs=S,
                                 num_minibatches=mb.num_minibatches)
  b = refcpu.sparse_dense_matmul(ref.row_pointers["t"], ref.embedding_ids["t"],
                                 ref.sample_ids["t"], ref.gains["t"], table,
                                 batch, num_sc_per_device=S, num_scs=S)
  np.testing.assert_array_equal(a, b)


def test_single_host_forward_and_backward_facts():
  """lib/nn/tests/minibatching_test.py:322-398 restated: limits of 2 ids
  and 2 unique ids force minibatches; with no id dropped, the lookup over a
  row-initialised table gives the sum of each sample's ids and SGD with unit
  gradients lowers every row by lr times its count. (The reference runs
  this on 4 SparseCores per chip; here S = 4 on one device, with limits
  that drop nothing.)"""
  rng = np.random.RandomState(2025)
  batch, vocab, dim, lr = 16, 2048, 16, 0.01
  feats = [_random_rows(rng, batch, vocab, 20)]
  # MOD sharding of a row-initialised table (utils.shard_emb_table).
  S = 4
  specs = [spec("feature_a", "table_a", max_ids=6, max_unique=6, batch=batch,
                vocab=vocab)]
  res = refcpu.preprocess(feats, None, specs, 1, 1, num_sc_per_device=S,
                          enable_minibatching=True, allow_id_dropping=True)
  assert res.num_minibatches > 1
  assert res.dropped_id_count["table_a"] == 0
  logical = np.arange(vocab, dtype=np.float32)
  phys = np.empty(vocab, np.float32)
  per = vocab // S
  phys[(logical.astype(int) % S) * per + logical.astype(int) // S] = logical
  table = np.repeat(phys[:, None], dim, axis=1)
  args = (res.row_pointers["table_a"], res.embedding_ids["table_a"],
          res.sample_ids["table_a"], res.gains["table_a"])
  act = refcpu.sparse_dense_matmul(*args, table, batch, num_sc_per_device=S,
                                   num_scs=S,
                                   num_minibatches=res.num_minibatches)
  np.testing.assert_allclose(
      act, np.repeat(np.array([r.sum() for r in feats[0]], np.float32)[:, None],
                     dim, axis=1), rtol=1e-6)
  new = refcpu.sparse_dense_matmul_grad(
      *args, np.ones((batch, dim), np.float32), table, learning_rate=lr,
      num_sc_per_device=S, num_scs=S, num_minibatches=res.num_minibatches)
  counts = np.bincount(np.concatenate(list(feats[0])), minlength=vocab)
  exp_logical = logical - lr * counts
  exp = np.empty(vocab, np.float32)
  exp[(logical.astype(int) % S) * per + logical.astype(int) // S] = exp_logical
  np.testing.assert_allclose(new, np.repeat(exp[:, None], dim, axis=1),
                             rtol=1e-6)


def test_buffer_sizes_with_minibatching():
  """ComputeTheoreticalMaxCooBufferSize (input_preprocessing_util.cc:
  244-255): 64 times the bound without minibatching."""
  lib = refcpu.lib()
  assert lib.ref_theoretical_max_coo_buffer_size_ex(16, 1, 4, 1) == \
      64 * lib.ref_theoretical_max_coo_buffer_size(16, 1, 4)
  assert lib.ref_coo_buffer_size_per_device_ex(16, 1024, 1, 4, 1) == 1024
  assert lib.ref_coo_buffer_size_per_device_ex(16, 1024, 1, 4, 0) == -1
