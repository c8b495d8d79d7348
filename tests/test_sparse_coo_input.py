"""Sparse COO input (preprocess_sparse_dense_matmul_sparse_coo_input and
embedding.preprocess_sparse_dense_matmul_input_from_sparse_tensor).

The reference's tests (lib/core/tests/sparse_coo_input_preprocessing_test.py
:84-186 16x16 ids on 4 devices x 4 SparseCores, :188-280 2400 rows of which
every 150th holds id 0, :1354-1460 the same 16x16 case on another spec)
require the COO entry to give exactly what the numpy entry gives for the same
ids with unit weights; so do these, on the GPU, and both are checked bit for
bit against the CPU oracle. On the CPU: the row splits against a direct
restatement of ConstructRowPointers (sparse_coo_input_batch.cc:30-66, one
pass over the row indices), and the rejected inputs.
"""

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip
from jax_tpu_embedding.sparsecore.lib.nn import embedding
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from oracle import refcpu

STACK = "one_table_to_rule_them_all"


def _row_pointers_loop(rows, batch):
  """ConstructRowPointers as a loop: before entry i, push i for every row up
  to rows[i]; then N up to batch."""
  out, r = [], 0
  for i, row in enumerate(rows):
    while r <= row:
      out.append(i)
      r += 1
  while r <= batch:
    out.append(len(rows))
    r += 1
  return np.array(out, np.int64)


def _random_coo(rng, batch, width, density):
  mask = rng.random((batch, width)) < density
  rows, cols = np.nonzero(mask)
  vals = rng.integers(0, 1000, size=rows.size).astype(np.int32)
  return np.stack([rows, cols], 1).astype(np.int64), vals


@pytest.mark.parametrize("seed", range(6))
def test_row_splits_match_construct_row_pointers(seed):
  rng = np.random.default_rng(seed)
  batch = int(rng.integers(1, 60))
  idx, vals = _random_coo(rng, batch, 7, [0.0, 0.05, 0.3, 0.9][seed % 4])
  r = pip.sparse_coo_to_ragged(idx, vals, [batch, 7])
  np.testing.assert_array_equal(r.row_splits,
                                _row_pointers_loop(idx[:, 0], batch))
  np.testing.assert_array_equal(r.values, vals)


@pytest.mark.parametrize("indices,message", [
    ([(1, 0), (0, 1)], "row-major"),
    ([(0, 2), (0, 1)], "row-major"),
    ([(0, 1), (0, 1)], "row-major"),
    ([(0, 0), (6, 0)], "outside"),
    ([(-1, 0)], "outside"),
])
def test_rejects_unsorted_or_out_of_range(indices, message):
  with pytest.raises(ValueError, match=message):
    pip.sparse_coo_to_ragged(indices, [1] * len(indices), [6, 10])


def _spec(vocab, dim, batch, input_width, max_ids=64, buffer=None):
  """A one-table stack laid out as the reference test's specs are
  (sparse_coo_input_preprocessing_test.py:35-81)."""
  opt = embedding_spec.SGDOptimizerSpec(learning_rate=0.001)
  table = embedding_spec.TableSpec(
      vocabulary_size=vocab, embedding_dim=dim, initializer=None,
      optimizer=opt, combiner="sum", name="table_b",
      max_ids_per_partition=max_ids, max_unique_ids_per_partition=max_ids,
      _setting_in_stack=embedding_spec.TableSettingInStack(
          stack_name=STACK, padded_vocab_size=vocab, padded_embedding_dim=dim,
          row_offset_in_shard=0, shard_rotation=0),
      _stacked_table_spec=embedding_spec.StackedTableSpec(
          stack_name=STACK, stack_vocab_size=vocab, stack_embedding_dim=dim,
          optimizer=opt, combiner="sum", total_sample_count=batch,
          max_ids_per_partition=max_ids,
          max_unique_ids_per_partition=max_ids,
          suggested_coo_buffer_size_per_device=buffer))
  return embedding_spec.FeatureSpec(
      table_spec=table, input_shape=[batch, input_width],
      output_shape=[batch, dim], name="feature_spec_b",
      _id_transformation=embedding_spec.FeatureIdTransformation(
          row_offset=0, col_offset=0, col_shift=0))


def _full_16x16():
  indices = [(i, j) for i in range(16) for j in range(16)]
  values = list(range(256))
  dense = np.arange(256, dtype=np.int32).reshape(16, 16)
  return indices, values, [16, 512], dense, np.ones((16, 16), np.float32)


def _every_150th_row():
  indices = [(i, 0) for i in range(0, 2251, 150)]
  values = [0] * len(indices)
  ragged = np.empty(2400, dtype=object)
  weights = np.empty(2400, dtype=object)
  for i in range(2400):
    ragged[i] = np.array([0] if i % 150 == 0 else [], np.int32)
    weights[i] = np.ones(len(ragged[i]), np.float32)
  return indices, values, [2400, 1], ragged, weights


CASES = {
    "full_16x16": (_full_16x16, dict(vocab=512, dim=8, batch=16,
                                     input_width=16)),
    "every_150th_row": (_every_150th_row, dict(
        vocab=512, dim=8, batch=2400, input_width=1, max_ids=150,
        buffer=1000)),
}


def _compare(got, exp, L, S):
  """Row pointers everywhere, the COO buffers on each segment's
  [0, row_pointers[-1]) (lib/core/tests/test_utils.py:19-43)."""
  rp_g, rp_e = (np.asarray(got[0]).reshape(-1),
                np.asarray(exp[0]).reshape(-1))
  np.testing.assert_array_equal(rp_g, rp_e)
  for g, e in zip(got[1:4], exp[1:4]):
    g, e = np.asarray(g).reshape(-1), np.asarray(e).reshape(-1)
    for seg, (rs, gs, es) in enumerate(zip(np.split(rp_e, L * S),
                                           np.split(g, L * S),
                                           np.split(e, L * S))):
      n = int(rs[-1])
      np.testing.assert_array_equal(gs[:n].view(np.int32),
                                    es[:n].view(np.int32), err_msg=str(seg))


def test_oracle_accepts_ragged_ids_like_ragged_rows():
  """The oracle reads RaggedIds (values + row splits) as the same ragged
  input as a list of rows."""
  indices, values, shape, ragged, weights = _every_150th_row()
  fs = _spec(**CASES["every_150th_row"][1])
  a = refcpu.preprocess([pip.sparse_coo_to_ragged(indices, values, shape)],
                        None, [fs], 4, 4, num_sc_per_device=4)
  b = refcpu.preprocess([ragged], [weights], [fs], 4, 4, num_sc_per_device=4)
  np.testing.assert_array_equal(a.row_pointers[STACK], b.row_pointers[STACK])
  _compare([a.row_pointers[STACK], a.embedding_ids[STACK],
            a.sample_ids[STACK], a.gains[STACK]],
           [b.row_pointers[STACK], b.embedding_ids[STACK],
            b.sample_ids[STACK], b.gains[STACK]], 4, 4)


def _gpu():
  torch = pytest.importorskip("torch")
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  return torch


def _cpu(x):
  return x.cpu().numpy() if hasattr(x, "cpu") else np.asarray(x)


@pytest.mark.gpu
@pytest.mark.parametrize("has_leading_dimension", [False, True])
@pytest.mark.parametrize("case", sorted(CASES))
def test_sparse_coo_entry_equals_numpy_entry(case, has_leading_dimension):
  _gpu()
  make, kw = CASES[case]
  indices, values, shape, features, weights = make()
  fs = _spec(**kw)
  common = dict(local_device_count=4, global_device_count=4,
                num_sc_per_device=4, sharding_strategy=pip.ShardingStrategy.MOD,
                has_leading_dimension=has_leading_dimension,
                allow_id_dropping=False, batch_number=42)
  sparse = pip.preprocess_sparse_dense_matmul_sparse_coo_input(
      [indices], [values], [shape], [fs], **common)
  raw = pip.preprocess_sparse_dense_matmul_input([features], [weights], [fs],
                                                 **common)
  got = [_cpu(x[STACK]) for x in sparse[:4]]
  exp = [_cpu(x[STACK]) for x in raw[:4]]
  if has_leading_dimension:
    assert got[0].shape[0] == 4
  _compare(got, exp, 4, 4)
  ref = refcpu.preprocess([pip.sparse_coo_to_ragged(indices, values, shape)],
                          None, [fs], 4, 4, num_sc_per_device=4)
  _compare(got, [ref.row_pointers[STACK], ref.embedding_ids[STACK],
                 ref.sample_ids[STACK], ref.gains[STACK]], 4, 4)
  for k in ("max_ids_per_partition", "max_unique_ids_per_partition"):
    np.testing.assert_array_equal(getattr(sparse[5], k)[STACK],
                                  getattr(raw[5], k)[STACK])


@pytest.mark.gpu
def test_embedding_entry_from_sparse_tensor_trains_like_ragged():
  """embedding.preprocess_sparse_dense_matmul_input_from_sparse_tensor with
  device tensors (indices, values on the GPU) gives the CSR, the stats and
  the forward activations of the ragged entry."""
  torch = _gpu()
  rng = np.random.default_rng(3)
  batch, vocab = 300, 4000
  tables = [embedding_spec.TableSpec(
      name=f"t{k}", vocabulary_size=vocab, embedding_dim=16,
      initializer=embedding_spec.normal(0.1),
      optimizer=embedding_spec.SGDOptimizerSpec(0.01), combiner=c,
      max_ids_per_partition=1 << 16, max_unique_ids_per_partition=1 << 16)
            for k, c in enumerate(("sum", "mean"))]
  feats = [embedding_spec.FeatureSpec(
      name=f"f{k}", table_spec=t, input_shape=[batch, 9],
      output_shape=[batch, 16]) for k, t in enumerate(tables)]
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  coo, ragged = [], []
  for _ in feats:
    idx, vals = _random_coo(rng, batch, 9, 0.4)
    vals = vals % vocab
    coo.append((torch.from_numpy(idx).cuda(), torch.from_numpy(vals).cuda(),
                np.array([batch, 9])))
    ragged.append(pip.sparse_coo_to_ragged(idx, vals, [batch, 9]))
  pre_s, stats_s = embedding.preprocess_sparse_dense_matmul_input_from_sparse_tensor(
      [c[0] for c in coo], [c[1] for c in coo], [c[2] for c in coo], feats,
      1, 1, num_sc_per_device=1)
  pre_r, stats_r = embedding.preprocess_sparse_dense_matmul_input(
      ragged, None, feats, 1, 1, num_sc_per_device=1)
  for name in pre_r.sparse_dense_matmul_input.lhs_row_pointers:
    got = [_cpu(x[name]) for x in pre_s.sparse_dense_matmul_input]
    exp = [_cpu(x[name]) for x in pre_r.sparse_dense_matmul_input]
    _compare(got, exp, 1, 1)
    np.testing.assert_array_equal(stats_s.max_ids_per_partition[name],
                                  stats_r.max_ids_per_partition[name])
  variables = embedding.init_embedding_variables(0, tables,
                                                 num_sparsecore_per_device=1)
  a_s = embedding.tpu_sparse_dense_matmul(pre_s, variables, feats,
                                          global_device_count=1,
                                          num_sc_per_device=1)
  a_r = embedding.tpu_sparse_dense_matmul(pre_r, variables, feats,
                                          global_device_count=1,
                                          num_sc_per_device=1)
  for x, y in zip(a_s, a_r):
    np.testing.assert_array_equal(x.cpu().numpy(), y.cpu().numpy())
