"""GPU parity: libscemb.so (through the drop-in API) against the CPU oracle.

Preprocessing must match bit for bit on the region the reference's own tests
compare (each segment's [0, row_pointers[-1]), lib/core/tests/
test_utils.py:19-43) plus all stats. Forward activations and updated tables /
accumulators must match within rtol 1e-5, atol 1e-6 (the tolerance BASELINE
states for fp32).
"""

import zlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


@pytest.fixture(scope="module", autouse=True)
def _gpu():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  torch.cuda.set_device(0)


from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr as fwd_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as adagrad_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd as sgd_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import table_stacking  # pylint: disable=g-import-not-at-top,wrong-import-position
from oracle import refcpu  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore import _native  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device  # pylint: disable=g-import-not-at-top,wrong-import-position


def _zipf(rng, a, vocab, size):
  out = np.empty(size, np.int64)
  filled = 0
  while filled < size:
    k = rng.zipf(a, size=2 * (size - filled) + 16)
    k = k[k <= vocab]
    take = min(size - filled, len(k))
    out[filled:filled + take] = k[:take] - 1
    filled += take
  return out.astype(np.int32)


def _make_specs(num_tables, vocabs, dims, combiner, optimizer, batch,
                features_per_table=1, max_ids=None):
  tables = [
      embedding_spec.TableSpec(
          name=f"table_{t}", vocabulary_size=int(vocabs[t]),
          embedding_dim=int(dims[t]), initializer=embedding_spec.zeros,
          optimizer=optimizer, combiner=combiner,
          max_ids_per_partition=max_ids or 1 << 20,
          max_unique_ids_per_partition=max_ids or 1 << 20)
      for t in range(num_tables)
  ]
  feats = []
  for t in range(num_tables):
    for k in range(features_per_table):
      feats.append(embedding_spec.FeatureSpec(
          name=f"feature_{t}_{k}", table_spec=tables[t],
          input_shape=[batch, 1], output_shape=[batch, int(dims[t])]))
  return tables, feats


def _stack(feats, names, global_device_count, num_sc, limit=1 << 20, **kw):
  """stack_tables with explicit stack limits (the default for a multi-table
  stack is 256, table_stacking.py:616-645)."""
  table_stacking.stack_tables(
      feats, names, global_device_count, num_sc,
      stack_to_max_ids_per_partition=lambda n, b: limit,
      stack_to_max_unique_ids_per_partition=lambda n, b: limit, **kw)


def _ragged(rng, batch, lo, hi, vocab, zipf_a=None):
  lens = rng.integers(lo, hi + 1, size=batch)
  rows = []
  for n in lens:
    if zipf_a:
      rows.append(_zipf(rng, zipf_a, vocab, int(n)))
    else:
      rows.append(rng.integers(0, vocab, size=int(n)).astype(np.int32))
  arr = np.empty(batch, dtype=object)
  for i, r in enumerate(rows):
    arr[i] = r
  return arr


def _weights_like(rng, ragged):
  arr = np.empty(len(ragged), dtype=object)
  for i, r in enumerate(ragged):
    arr[i] = rng.uniform(0, 1, size=len(r)).astype(np.float32)
  return arr


def _compare_preprocessing(features, weights, feature_specs, num_sc, *,
                           allow_id_dropping=False, local_device_count=1,
                           global_device_count=1):
  got = pip.preprocess_sparse_dense_matmul_input(
      features, weights, feature_specs, local_device_count,
      global_device_count, num_sc_per_device=num_sc,
      allow_id_dropping=allow_id_dropping)
  rps, eids, sids, gns, _, stats = got
  ref = refcpu.preprocess(features, weights, feature_specs,
                          local_device_count, global_device_count,
                          num_sc_per_device=num_sc,
                          allow_id_dropping=allow_id_dropping)
  segments = local_device_count * num_sc
  for name in ref.row_pointers:
    rp = rps[name].cpu().numpy()
    np.testing.assert_array_equal(rp, ref.row_pointers[name], err_msg=name)
    for got_d, exp_d in ((eids, ref.embedding_ids), (sids, ref.sample_ids),
                         (gns, ref.gains)):
      g = got_d[name].cpu().numpy()
      e = exp_d[name]
      assert g.shape == e.shape
      for seg, (rp_s, g_s, e_s) in enumerate(zip(
          np.split(rp, segments), np.split(g, segments),
          np.split(e, segments))):
        n = int(rp_s[-1])
        np.testing.assert_array_equal(
            g_s[:n].view(np.int32), e_s[:n].view(np.int32),
            err_msg=f"{name} segment {seg}")
    np.testing.assert_array_equal(stats.max_ids_per_partition[name],
                                  ref.max_ids_per_partition[name])
    np.testing.assert_array_equal(stats.max_unique_ids_per_partition[name],
                                  ref.max_unique_ids_per_partition[name])
    np.testing.assert_array_equal(stats.required_buffer_sizes[name],
                                  ref.required_buffer_sizes[name])
    assert stats.dropped_id_count[name] == ref.dropped_id_count[name]
  return got, ref


@pytest.mark.parametrize("combiner", ["sum", "mean", "sqrtn"])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("num_sc", [1, 2, 4])
def test_preprocess_ragged_stacked(combiner, weighted, num_sc):
  rng = np.random.default_rng(
      zlib.crc32(f"{combiner}-{weighted}-{num_sc}".encode()))
  batch = 64
  vocabs = [1000, 37, 5000]
  _, feats = _make_specs(3, vocabs, [16, 16, 16], combiner,
                         embedding_spec.SGDOptimizerSpec(0.01), batch,
                         features_per_table=2)
  _stack(feats, ["table_0", "table_1", "table_2"], 1, num_sc)
  features = [
      _ragged(rng, batch, 0, 12, vocabs[i // 2], zipf_a=1.2 if i % 2 else None)
      for i in range(len(feats))
  ]
  weights = [_weights_like(rng, f) for f in features] if weighted else None
  _compare_preprocessing(features, weights, feats, num_sc)


def test_preprocess_dense_dropping_and_rotation():
  rng = np.random.default_rng(7)
  batch = 128
  _, feats = _make_specs(2, [4000, 300], [8, 8], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch,
                         max_ids=6)
  _stack(feats, ["table_0", "table_1"], 1, 4, limit=6, rotation=1)
  features = [_zipf(rng, 1.1, 4000, batch * 5).reshape(batch, 5),
              rng.integers(0, 300, size=(batch, 3)).astype(np.int32)]
  (_, _, _, _, _, stats), ref = _compare_preprocessing(
      features, None, feats, 4, allow_id_dropping=True)
  name = feats[0].table_spec.stacked_table_spec.stack_name
  assert stats.dropped_id_count[name] == ref.dropped_id_count[name] > 0


def test_preprocess_limit_exceeded_raises():
  rng = np.random.default_rng(3)
  _, feats = _make_specs(1, [100], [8], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), 32, max_ids=2)
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  with pytest.raises(RuntimeError):
    pip.preprocess_sparse_dense_matmul_input(
        [rng.integers(0, 100, size=(32, 4)).astype(np.int32)], None, feats, 1,
        1, num_sc_per_device=1)


def test_preprocess_multi_device_layout():
  """L = 2 local devices, G = 2, S = 2: split-then-stack over devices."""
  rng = np.random.default_rng(11)
  batch = 32
  _, feats = _make_specs(2, [500, 80], [8, 8], "mean",
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  _stack(feats, ["table_0", "table_1"], 2, 2)
  features = [_ragged(rng, batch, 1, 6, 500), _ragged(rng, batch, 1, 3, 80)]
  _compare_preprocessing(features, None, feats, 2, local_device_count=2,
                         global_device_count=2)


def _csr_from_oracle(features, weights, feats, num_sc):
  ref = refcpu.preprocess(features, weights, feats, 1, 1,
                          num_sc_per_device=num_sc)
  name = next(iter(ref.row_pointers))
  return name, ref


def _entry_count(rp, num_sc):
  """Valid entries of a CSR: per segment, partition p holds
  [roundup8(rp[p-1]), rp[p])."""
  total = 0
  for seg in np.split(np.asarray(rp), num_sc):
    start = 0
    for end in seg:
      total += max(0, int(end) - start)
      start = max(start, (int(end) + 7) // 8 * 8)
  return total


def _fwd_bind(ref, name, table_t, batch, num_sc, view=None,
              num_entries=None):
  return fwd_prim.tpu_sparse_dense_matmul_csr_primitive.bind(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], 1, table_t, device_batch_size=batch,
      max_ids_per_partition=1 << 20, max_unique_ids_per_partition=1 << 20,
      num_sc_per_device=num_sc, lookup_view=view, csr_num_entries=num_entries)


def _view(ref, name, batch, rows, num_sc, num_entries=None):
  keep, c = _device.csr_operands(ref.row_pointers[name],
                                 ref.embedding_ids[name], ref.sample_ids[name],
                                 ref.gains[name], num_sc, num_sc,
                                 num_entries=num_entries)
  v = _native.build_sample_view(c, batch, rows)
  torch.cuda.synchronize()
  del keep
  return v


@pytest.mark.parametrize("dim", [1, 3, 8, 12, 64, 128, 256, 320, 520])
@pytest.mark.parametrize("num_sc", [1, 4])
@pytest.mark.parametrize("integer", [False, True])
def test_forward_matches_oracle(dim, num_sc, integer):
  """Forward through the CSR (grouping sort inside the call) and through a
  prebuilt sample view. Integer-valued tables with the sum combiner make
  every partial sum exact, so those results must agree bit for bit; float
  tables with the mean combiner are held to rtol 1e-5 / atol 1e-6."""
  rng = np.random.default_rng(dim * 7 + num_sc + (100 if integer else 0))
  batch = 96
  vocab = 2000
  _, feats = _make_specs(1, [vocab], [dim], "sum" if integer else "mean",
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  embedding.prepare_feature_specs_for_training(feats, 1, num_sc)
  # Integer cases: one id per sample (one-hot kernels), float: 0-40 ids.
  features = [_ragged(rng, batch, 1 if integer else 0, 1 if integer else 40,
                      vocab, zipf_a=1.1)]
  name, ref = _csr_from_oracle(features, None, feats, num_sc)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  if integer:
    table = rng.integers(-8, 9, size=(rows, dim)).astype(np.float32)
  else:
    table = rng.normal(0, 0.01, size=(rows, dim)).astype(np.float32)
  if dim == 1:
    table = table.reshape(rows)
  table_t = torch.from_numpy(table).cuda()
  # The entry count (known to the preprocessing) selects the one-hot kernel
  # variants for the one-id-per-sample cases.
  count = _entry_count(ref.row_pointers[name], num_sc)
  act = _fwd_bind(ref, name, table_t, batch, num_sc,
                  num_entries=count).cpu().numpy()
  act_v = _fwd_bind(ref, name, table_t, batch, num_sc,
                    view=_view(ref, name, batch, rows, num_sc, count),
                    num_entries=count).cpu().numpy()
  exp = refcpu.sparse_dense_matmul(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], table, batch, num_sc_per_device=num_sc, num_scs=num_sc)
  # Both routes feed the same kernel the same stream: identical bits.
  np.testing.assert_array_equal(act, act_v)
  if integer:
    np.testing.assert_array_equal(act, exp)
  else:
    np.testing.assert_allclose(act, exp, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("dim", [4, 128, 300])
def test_forward_long_rows_and_empty_rows(dim):
  """Activation rows of up to 3000 entries span many 256-entry blocks (the
  cross-block partial path); every third row, the first rows and the last
  rows have no entries and must come out zero."""
  rng = np.random.default_rng(dim)
  batch = 64
  vocab = 500
  _, feats = _make_specs(1, [vocab], [dim], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch,
                         max_ids=1 << 16)
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  arr = np.empty(batch, dtype=object)
  for i in range(batch):
    n = 0 if (i % 3 == 0 or i < 2 or i >= batch - 3) else int(
        rng.integers(1, 3000))
    arr[i] = rng.integers(0, vocab, size=n).astype(np.int32)
  name, ref = _csr_from_oracle([arr], None, feats, 1)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  table = rng.integers(-4, 5, size=(rows, dim)).astype(np.float32)
  table_t = torch.from_numpy(table).cuda()
  exp = refcpu.sparse_dense_matmul(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], table, batch, num_sc_per_device=1, num_scs=1)
  for view in (None, _view(ref, name, batch, rows, 1)):
    # Poison the output allocation first: empty rows must be written.
    junk = torch.full((batch, dim), float("nan"), device="cuda")
    del junk
    act = _fwd_bind(ref, name, table_t, batch, 1, view=view).cpu().numpy()
    np.testing.assert_array_equal(act, exp)
    assert not act[0].any() and not act[-1].any()


@pytest.mark.parametrize("dim", [8, 128])
def test_forward_runs_ending_at_block_edges(dim):
  """Activation rows laid out so that runs of the sorted stream end exactly
  on 256-entry block edges: a run that starts in one block and ends on the
  last entry of the next, one that fills a block, one that spans three
  blocks, single entries at an edge. Ids are distinct within a row, so every
  id is one entry; integer tables make the sums exact, so the forward must
  equal the oracle bit for bit through both routes."""
  rng = np.random.default_rng(dim + 11)
  lengths = [200, 312, 256, 100, 412, 600, 1, 423, 0, 255, 1, 700, 40, 216,
             256, 257, 255]
  batch = 48
  lengths += [int(x) for x in rng.integers(0, 300, size=batch - len(lengths))]
  vocab = 4096
  _, feats = _make_specs(1, [vocab], [dim], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch,
                         max_ids=1 << 16)
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  arr = np.empty(batch, dtype=object)
  for i, n in enumerate(lengths):
    arr[i] = rng.permutation(vocab)[:n].astype(np.int32)
  ends = np.cumsum(lengths)
  assert 512 in ends and 1280 in ends and 2304 in ends and 2560 in ends
  name, ref = _csr_from_oracle([arr], None, feats, 1)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  table = rng.integers(-4, 5, size=(rows, dim)).astype(np.float32)
  table_t = torch.from_numpy(table).cuda()
  exp = refcpu.sparse_dense_matmul(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], table, batch, num_sc_per_device=1, num_scs=1)
  for view in (None, _view(ref, name, batch, rows, 1)):
    act = _fwd_bind(ref, name, table_t, batch, 1, view=view).cpu().numpy()
    np.testing.assert_array_equal(act, exp)


def test_forward_empty_batch_is_zero():
  rng = np.random.default_rng(2)
  batch = 40
  _, feats = _make_specs(1, [100], [16], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  arr = np.empty(batch, dtype=object)
  for i in range(batch):
    arr[i] = np.zeros(0, np.int32)
  name, ref = _csr_from_oracle([arr], None, feats, 1)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  table = torch.from_numpy(rng.normal(size=(rows, 16)).astype(np.float32))
  act = _fwd_bind(ref, name, table.cuda(), batch, 1).cpu().numpy()
  assert act.shape == (batch, 16) and not act.any()


def _run_grad(optimizer, csr, grad, table0, acc0, lr, lo, hi, num_sc,
              sorted_by_row=False):
  """Runs the GPU primitive and the oracle; returns (got, expected) pairs.
  `sorted_by_row` lets the kernel read the CSR in place (one segment); the
  entry count is passed as the preprocessing would."""
  table = torch.from_numpy(table0.copy()).cuda()
  count = _entry_count(csr[0], num_sc)
  if optimizer == "sgd":
    out = sgd_prim.tpu_sparse_dense_matmul_grad_with_sgd_primitive.bind(
        *csr, 1, table, torch.from_numpy(grad).cuda(), lr,
        max_ids_per_partition=1 << 20, max_unique_ids_per_partition=1 << 20,
        min_value=lo, max_value=hi, num_sc_per_device=num_sc,
        csr_sorted_by_row=sorted_by_row, csr_num_entries=count)
    assert out is table
    exp_t = refcpu.sparse_dense_matmul_grad(
        *csr, grad, table0, None, learning_rate=lr,
        num_sc_per_device=num_sc, num_scs=num_sc, min_value=lo, max_value=hi)
    return [(table.cpu().numpy(), exp_t)]
  acc = torch.from_numpy(acc0.copy()).cuda()
  out_t, out_a = (
      adagrad_prim.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
          *csr, 1, table, acc, torch.from_numpy(grad).cuda(), np.float32(lr),
          max_ids_per_partition=1 << 20, max_unique_ids_per_partition=1 << 20,
          min_value=lo, max_value=hi, num_sc_per_device=num_sc,
          csr_sorted_by_row=sorted_by_row, csr_num_entries=count))
  assert out_t is table and out_a is acc
  exp_t, exp_a = refcpu.sparse_dense_matmul_grad(
      *csr, grad, table0, acc0, learning_rate=lr, num_sc_per_device=num_sc,
      num_scs=num_sc, min_value=lo, max_value=hi)
  return [(table.cpu().numpy(), exp_t), (acc.cpu().numpy(), exp_a)]


@pytest.mark.parametrize("optimizer", ["sgd", "adagrad"])
@pytest.mark.parametrize("dim", [1, 8, 24, 128, 256, 300])
@pytest.mark.parametrize("num_sc,sorted_by_row", [(1, False), (1, True),
                                                  (2, False), (2, True)])
@pytest.mark.parametrize("clip", [False, True])
def test_grad_hot_rows_exact(optimizer, dim, num_sc, sorted_by_row, clip):
  """Long runs of hot rows (Zipf 1.05 over 300 rows) cross block boundaries
  and use the cross-block reduction. Integer-valued gradients with unit
  gains make every partial sum exact, so the result may not depend on
  summation order: GPU and oracle must agree bit for bit. With one segment
  and sorted_by_row the kernel reads the CSR in place (with two segments the
  flag must be ignored and the entries sorted)."""
  rng = np.random.default_rng(dim * 13 + num_sc + (7 if clip else 0))
  batch = 4096 if dim <= 128 else 512
  vocab = 300
  _, feats = _make_specs(1, [vocab], [dim], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  embedding.prepare_feature_specs_for_training(feats, 1, num_sc)
  # Clipped cases use one id per sample (the kernels' one-hot variants),
  # unclipped ones 1-8 ids (the multi-hot variants).
  hi_len = 1 if clip else 8
  features = [_ragged(rng, batch, 1, hi_len, vocab, zipf_a=1.05)]
  name, ref = _csr_from_oracle(features, None, feats, num_sc)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  shape = (rows,) if dim == 1 else (rows, dim)
  table0 = rng.normal(0, 0.01, size=shape).astype(np.float32)
  acc0 = np.full(shape, 0.1, np.float32)
  grad = rng.integers(-3, 4, size=(batch,) if dim == 1 else
                      (batch, dim)).astype(np.float32)
  lo, hi = (-0.005, 0.005) if clip else (None, None)
  csr = (ref.row_pointers[name], ref.embedding_ids[name],
         ref.sample_ids[name], ref.gains[name])
  for got, exp in _run_grad(optimizer, csr, grad, table0, acc0, 0.05, lo, hi,
                            num_sc, sorted_by_row):
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("optimizer", ["sgd", "adagrad"])
@pytest.mark.parametrize("combiner", ["sum", "mean", "sqrtn"])
@pytest.mark.parametrize("dim", [8, 64, 128])
@pytest.mark.parametrize("num_sc", [1, 4])
def test_grad_float_matches_oracle(optimizer, combiner, dim, num_sc):
  """Float gains and gradients, short runs: within rtol 1e-5 / atol 1e-6."""
  rng = np.random.default_rng(zlib.crc32(
      f"{optimizer}-{combiner}-{dim}-{num_sc}".encode()))
  batch = 2048
  vocab = 200_000
  _, feats = _make_specs(1, [vocab], [dim], combiner,
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  embedding.prepare_feature_specs_for_training(feats, 1, num_sc)
  features = [_ragged(rng, batch, 1, 30, vocab)]
  weights = [_weights_like(rng, features[0])]
  name, ref = _csr_from_oracle(features, weights, feats, num_sc)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  table0 = rng.normal(0, 0.01, size=(rows, dim)).astype(np.float32)
  acc0 = np.full((rows, dim), 0.1, np.float32)
  grad = rng.normal(0, 1, size=(batch, dim)).astype(np.float32)
  csr = (ref.row_pointers[name], ref.embedding_ids[name],
         ref.sample_ids[name], ref.gains[name])
  for got, exp in _run_grad(optimizer, csr, grad, table0, acc0, 0.05, None,
                            None, num_sc, sorted_by_row=num_sc == 1):
    np.testing.assert_allclose(got, exp, rtol=RTOL, atol=ATOL)


def _hot_float_case(seed, batch=8192, dim=64):
  rng = np.random.default_rng(seed)
  _, feats = _make_specs(1, [40], [dim], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  features = [_zipf(rng, 1.2, 40, batch * 4).reshape(batch, 4)]
  name, ref = _csr_from_oracle(features, None, feats, 1)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  table0 = rng.normal(0, 0.01, size=(rows, dim)).astype(np.float32)
  acc0 = np.full((rows, dim), 0.1, np.float32)
  grad = rng.normal(0, 1, size=(batch, dim)).astype(np.float32)
  csr = (ref.row_pointers[name], ref.embedding_ids[name],
         ref.sample_ids[name], ref.gains[name])
  return csr, grad, table0, acc0


def test_grad_deterministic_and_modes_agree():
  """Float gradients on hot rows (runs of thousands of entries): repeated
  calls give identical bits, and reading the CSR in place gives the same
  bits as sorting a copy (same stream order, same blocks)."""
  csr, grad, table0, acc0 = _hot_float_case(17)
  runs = [_run_grad("adagrad", csr, grad, table0, acc0, 0.05, None, None, 1,
                    sorted_by_row=s) for s in (False, False, True, True)]
  for r in runs[1:]:
    for (got, _), (got0, _) in zip(r, runs[0]):
      np.testing.assert_array_equal(got, got0)


def test_grad_hot_float_close_to_float64():
  """The same hot-row case against a float64 restatement of the update.

  Each row gradient is an fp32 sum of up to ~20k terms, evaluated as
  sequential pieces of at most 64 entries added in a tree. The classical
  bound for such a sum is |err| <= (64 + log2(#pieces) + 1) * eps32 * sum|x|,
  below e = 3e-6 * sum|x|. The accumulator A = 0.1 + g^2 then errs by at
  most 2|g|e + e^2, and the table by at most lr * |d/dg g/sqrt(0.1+g^2)| * e
  <= lr * 0.1**-0.5 * e, each plus a few ulps of its own rounding."""
  csr, grad, table0, acc0 = _hot_float_case(23)
  (got_t, _), (got_a, _) = _run_grad("adagrad", csr, grad, table0, acc0, 0.05,
                                     None, None, 1, sorted_by_row=True)
  rp, eid, sid, gains = csr
  n = int(rp[0])
  terms = grad[sid[:n]].astype(np.float64) * gains[:n, None].astype(np.float64)
  g64 = np.zeros(table0.shape, np.float64)
  mag = np.zeros(table0.shape, np.float64)
  np.add.at(g64, eid[:n], terms)
  np.add.at(mag, eid[:n], np.abs(terms))
  touched = np.zeros(table0.shape[0], bool)
  touched[eid[:n]] = True
  a64 = acc0.astype(np.float64) + np.where(touched[:, None], g64 * g64, 0)
  t64 = table0.astype(np.float64) - np.where(
      touched[:, None], 0.05 * g64 / np.sqrt(a64), 0)
  e = 3e-6 * mag
  bound_a = 2 * np.abs(g64) * e + e * e + 4e-7 * a64
  bound_t = 0.05 * 0.1**-0.5 * e + 4e-7 * np.abs(t64) + 1e-9
  assert (np.abs(got_a - a64) <= bound_a).all()
  assert (np.abs(got_t - t64) <= bound_t).all()
  # The bound is not vacuous: typical errors sit well inside it and the
  # largest sums carry rounding at all.
  assert np.abs(got_a - a64).max() > 0


def test_unsorted_csr_declared_sorted_is_flagged():
  """A CSR whose entries are not ascending, passed with the sorted flag:
  the kernel reports SCEMB_STATUS_UNSORTED instead of failing silently; the
  same CSR without the flag is sorted and matches the oracle."""
  rng = np.random.default_rng(4)
  rows, dim, batch = 64, 8, 32
  n = 40
  eid = rng.integers(0, rows, size=n).astype(np.int32)
  sid = rng.integers(0, batch, size=n).astype(np.int32)
  assert (np.diff(eid) < 0).any()
  rp = np.full(8, n, np.int32)
  gains = np.ones(n, np.float32)
  grad = rng.integers(-3, 4, size=(batch, dim)).astype(np.float32)
  table0 = rng.normal(size=(rows, dim)).astype(np.float32)
  keep, c = _device.csr_operands(rp, eid, sid, gains, 1, 1,
                                 sorted_by_row=True)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  table = torch.from_numpy(table0.copy()).cuda()
  _native.sparse_dense_matmul_grad(c, torch.from_numpy(grad).cuda(), table,
                                   None, 0.1, batch, device_status=status)
  assert int(status.item()) & _native.STATUS_UNSORTED
  del keep
  (got, exp), = _run_grad("sgd", (rp, eid, sid, gains), grad, table0, None,
                          0.1, None, None, 1, sorted_by_row=False)
  np.testing.assert_array_equal(got, exp)


def test_end_to_end_api_feature_stacking_adagrad():
  """Two features on one table (feature stacking) + a second table, mean
  combiner, Adagrad through embedding.tpu_sparse_dense_matmul(_grad)."""
  rng = np.random.default_rng(5)
  batch = 256
  opt = embedding_spec.AdagradOptimizerSpec(learning_rate=0.01,
                                            initial_accumulator_value=0.1)
  tables, feats = _make_specs(2, [3000, 50000], [32, 32], "mean", opt, batch,
                              features_per_table=2)
  _stack(feats, ["table_0", "table_1"], 1, 1)
  features = [_ragged(rng, batch, 1, 20, t.vocabulary_size, zipf_a=1.2)
              for t in (tables[0], tables[0], tables[1], tables[1])]
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      features, None, feats, 1, 1, num_sc_per_device=1)
  name = feats[0].table_spec.stacked_table_spec.stack_name
  ref = refcpu.preprocess(features, None, feats, 1, 1, num_sc_per_device=1)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  table0 = rng.normal(0, 0.01, size=(rows, 32)).astype(np.float32)
  acc0 = np.full((rows, 32), 0.1, np.float32)
  variables = {name: embedding.EmbeddingVariables(
      torch.from_numpy(table0.copy()).cuda(),
      (torch.from_numpy(acc0.copy()).cuda(),))}
  acts = embedding.tpu_sparse_dense_matmul(pre, variables, feats,
                                           global_device_count=1,
                                           num_sc_per_device=1)
  stacked_exp = refcpu.sparse_dense_matmul(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], table0, 4 * batch, num_sc_per_device=1, num_scs=1)
  for k, a in enumerate(acts):
    np.testing.assert_allclose(a.cpu().numpy(),
                               stacked_exp[k * batch:(k + 1) * batch],
                               rtol=RTOL, atol=ATOL)
  grads = [rng.normal(0, 1, size=(batch, 32)).astype(np.float32)
           for _ in range(4)]
  out = embedding.tpu_sparse_dense_matmul_grad(
      [torch.from_numpy(g).cuda() for g in grads], pre, variables, feats,
      global_device_count=1, num_sc_per_device=1)
  exp_t, exp_a = refcpu.sparse_dense_matmul_grad(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], np.concatenate(grads), table0, acc0,
      learning_rate=0.01, num_sc_per_device=1, num_scs=1)
  np.testing.assert_allclose(out[name].table.cpu().numpy(), exp_t, rtol=RTOL,
                             atol=ATOL)
  np.testing.assert_allclose(out[name].slot[0].cpu().numpy(), exp_a,
                             rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("num_sc", [1, 2])
@pytest.mark.parametrize("integer", [True, False])
def test_fused_unstack_and_gradient_stack_match_copy_paths(num_sc, integer):
  """The embedding API writes activations straight into per-feature outputs
  and reads per-feature gradients in place (row blocks). Same results as the
  stacked-matrix path plus unstack_embedding_activations /
  stack_embedding_gradients: bit for bit with integer data (every sum is
  exact whatever the kernel layout), within rtol 1e-5 / atol 1e-6 with float
  data. Dims 12 (padded to 16: the padding columns are neither written nor
  read) and 16 share one stack; one feature takes only 10 of its 12 dims."""
  rng = np.random.default_rng(31 + num_sc + (5 if integer else 0))
  batch = 128
  opt = embedding_spec.AdagradOptimizerSpec(learning_rate=0.02,
                                            initial_accumulator_value=0.1)
  def specs(out_dim_f1):
    t0 = embedding_spec.TableSpec(
        name="t0", vocabulary_size=700, embedding_dim=12,
        initializer=embedding_spec.zeros, optimizer=opt, combiner="sum",
        max_ids_per_partition=1 << 16, max_unique_ids_per_partition=1 << 16)
    t1 = embedding_spec.TableSpec(
        name="t1", vocabulary_size=300, embedding_dim=16,
        initializer=embedding_spec.zeros, optimizer=opt, combiner="sum",
        max_ids_per_partition=1 << 16, max_unique_ids_per_partition=1 << 16)
    return [
        embedding_spec.FeatureSpec(name="f0", table_spec=t0,
                                   input_shape=[batch, 1],
                                   output_shape=[batch, 12]),
        embedding_spec.FeatureSpec(name="f1", table_spec=t0,
                                   input_shape=[batch, 1],
                                   output_shape=[batch, out_dim_f1]),
        embedding_spec.FeatureSpec(name="f2", table_spec=t1,
                                   input_shape=[batch, 1],
                                   output_shape=[batch, 16]),
    ]

  features = [_ragged(rng, batch, 1, 6, 700, zipf_a=1.1),
              _ragged(rng, batch, 0, 4, 700),
              _ragged(rng, batch, 1, 3, 300, zipf_a=1.3)]
  for out_dim_f1, check_grad in ((10, False), (12, True)):
    feats = specs(out_dim_f1)
    _stack(feats, ["t0", "t1"], 1, num_sc, limit=1 << 16)
    pre, _ = embedding.preprocess_sparse_dense_matmul_input(
        features, None, feats, 1, 1, num_sc_per_device=num_sc)
    name = feats[0].table_spec.stacked_table_spec.stack_name
    spec = feats[0].table_spec.stacked_table_spec
    shape = (spec.stack_vocab_size, spec.stack_embedding_dim)
    table0 = (rng.integers(-4, 5, size=shape) if integer else
              rng.normal(0, 0.01, size=shape)).astype(np.float32)

    def variables():
      return {name: embedding.EmbeddingVariables(
          torch.from_numpy(table0.copy()).cuda(),
          (torch.full(shape, 0.1, dtype=torch.float32, device="cuda"),))}

    v = variables()
    fused = embedding.tpu_sparse_dense_matmul(
        pre, v, feats, global_device_count=1, num_sc_per_device=num_sc)
    stacked = embedding.tpu_sparse_dense_matmul(
        pre, v, feats, global_device_count=1, num_sc_per_device=num_sc,
        perform_unstacking=False)
    copied = embedding.unstack_embedding_activations(stacked, feats, 1,
                                                     num_sc)
    for a, b in zip(fused, copied):
      assert tuple(a.shape) == tuple(b.shape)
      if integer:
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())
      else:
        np.testing.assert_allclose(a.cpu().numpy(), b.cpu().numpy(),
                                   rtol=RTOL, atol=ATOL)
    if not check_grad:
      continue
    grads = [torch.from_numpy(
        (rng.integers(-3, 4, size=(batch, fs.table_spec.embedding_dim))
         if integer else rng.normal(size=(batch, fs.table_spec.embedding_dim))
         ).astype(np.float32)).cuda() for fs in feats]
    v_fused, v_copy = variables(), variables()
    embedding.tpu_sparse_dense_matmul_grad(
        grads, pre, v_fused, feats, global_device_count=1,
        num_sc_per_device=num_sc)
    stacked_grads = embedding.stack_embedding_gradients(grads, feats, num_sc)
    embedding.tpu_sparse_dense_matmul_grad(
        stacked_grads, pre, v_copy, feats, global_device_count=1,
        num_sc_per_device=num_sc, perform_stacking=False)
    for x, y in ((v_fused[name].table, v_copy[name].table),
                 (v_fused[name].slot[0], v_copy[name].slot[0])):
      if integer:
        np.testing.assert_array_equal(x.cpu().numpy(), y.cpu().numpy())
      else:
        np.testing.assert_allclose(x.cpu().numpy(), y.cpu().numpy(),
                                   rtol=RTOL, atol=ATOL)
    # The stacking padding of the table (columns 12..15 of t0's rows) only
    # ever sees zero gradient.
    assert bool((v_fused[name].slot[0][:, 12:16] ==
                 v_copy[name].slot[0][:, 12:16]).all())


@pytest.mark.parametrize("num_sc", [1, 4])
def test_one_entry_per_row_view_matches_sorted_view(num_sc):
  """With at most one id per input row, the sample view built by placement
  (CSR_ONE_ENTRY_PER_ROW: count, scan, compaction) is bit for bit the view
  the radix sort builds, with empty rows (no id) and invalid entries among
  the samples, and the forward results agree bit for bit."""
  rng = np.random.default_rng(17 + num_sc)
  batch, vocab, dim = 512, 3000, 16
  tables, feats = _make_specs(2, [vocab, 700], [dim, dim], "sum",
                              embedding_spec.SGDOptimizerSpec(0.01), batch)
  _stack(feats, ["table_0", "table_1"], 1, num_sc)
  features = []
  for t in tables:
    rows = np.empty(batch, dtype=object)
    for i in range(batch):
      rows[i] = (np.array([rng.integers(0, t.vocabulary_size)], np.int32)
                 if rng.random() < 0.8 else np.zeros(0, np.int32))
    features.append(rows)
  name, ref = _csr_from_oracle(features, None, feats, num_sc)
  spec = feats[0].table_spec.stacked_table_spec
  bs, rows_ = spec.total_sample_count, spec.stack_vocab_size
  csr = (ref.row_pointers[name], ref.embedding_ids[name],
         ref.sample_ids[name], ref.gains[name].copy())
  # Two entries with an embedding id outside the table: skipped either way.
  bad = np.nonzero(csr[1] != np.iinfo(np.int32).max)[0][:2]
  csr[1][bad] = rows_ // num_sc + 5
  views = []
  for one in (False, True):
    keep, c = _device.csr_operands(*csr, num_sc, num_sc,
                                   one_entry_per_row=one)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    views.append((_native.build_sample_view(c, bs, rows_,
                                            device_status=status), status))
    torch.cuda.synchronize()
    del keep
  (v0, s0), (v1, s1) = views
  np.testing.assert_array_equal(v1.keys.cpu().numpy(), v0.keys.cpu().numpy())
  np.testing.assert_array_equal(v1.entries.cpu().numpy(),
                                v0.entries.cpu().numpy())
  assert int(s0.item()) == int(s1.item()) == _native.STATUS_BAD_ENTRY
  table = torch.from_numpy(
      rng.normal(size=(rows_, dim)).astype(np.float32)).cuda()
  acts = [_fwd_bind(ref, name, table, bs, num_sc, view=v).cpu().numpy()
          for v in (v0, v1)]
  np.testing.assert_array_equal(acts[0], acts[1])


def test_shared_row_in_one_entry_per_row_csr_is_flagged():
  """A CSR with two entries for one activation row, declared one entry per
  row: the placement reports SCEMB_STATUS_SHARED_ROW."""
  rp = np.full(8, 3, np.int32)
  eid = np.array([1, 2, 3], np.int32)
  sid = np.array([0, 5, 0], np.int32)
  gains = np.ones(3, np.float32)
  keep, c = _device.csr_operands(rp, eid, sid, gains, 1, 1,
                                 one_entry_per_row=True)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  _native.build_sample_view(c, 8, 16, device_status=status)
  assert int(status.item()) & _native.STATUS_SHARED_ROW
  del keep


@pytest.mark.parametrize("shared", [False, True])
def test_undeclared_csr_stream_is_the_stable_row_sort(shared):
  """A small CSR with padding, not declared one entry per row, with and
  without a row that holds two entries: the sample stream is the stable
  sort of the valid entries by activation row, the rest holds the unused
  key, and no status is raised for the shared row (nothing was declared)."""
  pad = np.iinfo(np.int32).max
  rp = np.full(8, 5, np.int32)
  eid = np.array([1, 2, 3, 4, 6, pad, pad, pad], np.int32)
  sid = np.array([0, 5, 7 if not shared else 0, 3, 6, pad, pad, pad],
                 np.int32)
  gains = np.array([1, 2, 3, 4, 5, np.nan, np.nan, np.nan], np.float32)
  batch, rows = 8, 16
  keep, c = _device.csr_operands(rp, eid, sid, gains, 1, 1)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  v = _native.build_sample_view(c, batch, rows, device_status=status)
  torch.cuda.synchronize()
  order = np.argsort(sid[:5], kind="stable")
  keys = v.keys.cpu().numpy()
  entries = v.entries.cpu().numpy()
  np.testing.assert_array_equal(keys[:5], sid[:5][order])
  np.testing.assert_array_equal(
      entries[:5], eid[:5][order].astype(np.uint64) |
      (gains[:5][order].view(np.uint32).astype(np.uint64) << np.uint64(32)))
  assert (keys[5:] == batch).all()
  assert int(status.item()) == 0
  del keep


@pytest.mark.parametrize("num_sc", [1, 2])
@pytest.mark.parametrize("weighted", [False, True])
def test_preprocessing_view_groups_like_the_csr_view(num_sc, weighted):
  """The sample view the preprocessing writes along with the CSR holds, for
  every activation row, the same entries as the view built from the CSR by
  sorting (only their order inside a row may differ), with ids dropped by
  the limits, duplicate ids merged and empty rows; the forward gives the
  same activations bit for bit on integer data."""
  rng = np.random.default_rng(23 + num_sc + (10 if weighted else 0))
  batch = 256
  tables, feats = _make_specs(2, [900, 4000], [8, 8], "sum",
                              embedding_spec.SGDOptimizerSpec(0.01), batch,
                              features_per_table=2)
  _stack(feats, ["table_0", "table_1"], 1, num_sc, limit=48)
  features = [_ragged(rng, batch, 0, 12, t.vocabulary_size, zipf_a=1.2)
              for t in (tables[0], tables[0], tables[1], tables[1])]
  weights = ([_weights_like(rng, f) for f in features] if weighted else None)
  pre, stats = embedding.preprocess_sparse_dense_matmul_input(
      features, weights, feats, 1, 1, num_sc_per_device=num_sc,
      allow_id_dropping=True)
  name = feats[0].table_spec.stacked_table_spec.stack_name
  assert sum(stats.id_drop_counters.values()) > 0
  spec = feats[0].table_spec.stacked_table_spec
  bs, rows = spec.total_sample_count, spec.stack_vocab_size
  got = pre.lookup_views[name]
  keep, c = _device.csr_operands(pre.lhs_row_pointers[name],
                                 pre.lhs_embedding_ids[name],
                                 pre.lhs_sample_ids[name],
                                 pre.lhs_gains[name], num_sc, num_sc)
  exp = _native.build_sample_view(c, bs, rows)
  torch.cuda.synchronize()
  del keep
  gk, ge = got.keys.cpu().numpy(), got.entries.cpu().numpy()
  ek, ee = exp.keys.cpu().numpy(), exp.entries.cpu().numpy()
  np.testing.assert_array_equal(gk, ek)
  og, oe = np.lexsort((ge, gk)), np.lexsort((ee, ek))
  np.testing.assert_array_equal(ge[og], ee[oe])
  table = torch.from_numpy(
      rng.integers(-4, 5, size=(rows, 8)).astype(np.float32)).cuda()
  csr = (pre.lhs_row_pointers[name], pre.lhs_embedding_ids[name],
         pre.lhs_sample_ids[name], pre.lhs_gains[name])
  acts = []
  for v in (got, exp):
    acts.append(fwd_prim.tpu_sparse_dense_matmul_csr_primitive.bind(
        *csr, 1, table, device_batch_size=bs, max_ids_per_partition=48,
        max_unique_ids_per_partition=48, num_sc_per_device=num_sc,
        lookup_view=v).cpu().numpy())
  if weighted:
    np.testing.assert_allclose(acts[0], acts[1], rtol=RTOL, atol=ATOL)
  else:
    np.testing.assert_array_equal(acts[0], acts[1])


@pytest.mark.parametrize("mapped", [False, True])
def test_one_entry_per_key_view_skips_the_combining_pass(mapped):
  """A one-hot stack's sample view declares that no key repeats: the
  forward then skips its cross-block combining launch. Its activations equal
  those of the same view without the declaration, bit for bit, through
  the dense output and through per-feature row blocks."""
  rng = np.random.default_rng(41)
  batch, rows_, dim = 5000, 3000, 32
  sid = rng.permutation(batch)[:4000].astype(np.int32)  # rows without ids
  eid = rng.integers(0, rows_, size=sid.size).astype(np.int32)
  gains = rng.uniform(0.5, 2.0, size=sid.size).astype(np.float32)
  order = np.lexsort((sid, eid))
  eid, sid, gains = eid[order], sid[order], gains[order]
  n = -(-sid.size // 8) * 8
  pad = n - sid.size
  eid = np.concatenate([eid, np.full(pad, 2**31 - 1, np.int32)])
  sid = np.concatenate([sid, np.full(pad, 2**31 - 1, np.int32)])
  gains = np.concatenate([gains, np.full(pad, np.nan, np.float32)])
  rp = np.full(8, 4000, np.int32)
  keep, c = _device.csr_operands(rp, eid, sid, gains, 1, 1,
                                 one_entry_per_row=True, num_entries=4000)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  view = _native.build_sample_view(c, batch, rows_, device_status=status)
  assert view.one_entry_per_key
  plain = _native.LookupView(view.keys, view.entries, batch, rows_,
                             view.num_entries)
  table = torch.from_numpy(
      rng.normal(size=(rows_, dim)).astype(np.float32)).cuda()
  outs = []
  for v in (view, plain):
    if mapped:
      blocks = [torch.full((2600, dim), 7.0, device="cuda"),
                torch.full((2400, dim), 7.0, device="cuda")]
      _native.sparse_dense_matmul_to_blocks(
          None, table, [(0, blocks[0], dim), (2600, blocks[1], dim)],
          batch, view=v, device_status=status)
      out = torch.cat(blocks)
    else:
      out = torch.full((batch, dim), 7.0, device="cuda")
      _native.sparse_dense_matmul(None, table, out, batch, view=v,
                                  device_status=status)
    outs.append(out.cpu().numpy())
  torch.cuda.synchronize()
  assert int(status.item()) == 0
  np.testing.assert_array_equal(outs[0], outs[1])
  expect = np.zeros((batch, dim), np.float32)
  expect[sid[:4000]] = (gains[:4000, None] *
                        table.cpu().numpy()[eid[:4000]])
  np.testing.assert_array_equal(outs[0], expect)
  del keep


def test_repeated_key_in_one_entry_per_key_view_is_flagged():
  """A view declared with no repeated key that has one spanning a block:
  the forward reports SCEMB_STATUS_SHARED_ROW."""
  batch, rows_, dim = 400, 16, 8
  # Every key twice; positions 255 and 256 (two blocks) share key 128.
  keys = ((np.arange(600) + 1) // 2).astype(np.uint32)
  entries = (np.arange(600, dtype=np.uint64) % rows_) | (
      np.uint64(np.float32(1.0).view(np.uint32)) << np.uint64(32))
  kt = torch.from_numpy(keys.view(np.int32)).cuda()
  et = torch.from_numpy(entries.view(np.int64)).cuda()
  view = _native.LookupView(kt, et, batch, rows_, 600,
                            one_entry_per_key=True)
  table = torch.ones(rows_, dim, device="cuda")
  out = torch.empty(batch, dim, device="cuda")
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  _native.sparse_dense_matmul(None, table, out, batch, view=view,
                              device_status=status)
  torch.cuda.synchronize()
  assert int(status.item()) & _native.STATUS_SHARED_ROW


def _expected_sample_stream(rp, eid, sid, gains, num_sc, bps, rpp):
  """The CSR's valid entries grouped by activation row, each row in CSR
  order (a stable sort by row), as (keys, packed entries) with the entry
  packed as (partition * rows_per_partition + id) | gain bits << 32."""
  rp = np.asarray(rp).reshape(num_sc, -1)
  eid, sid = np.asarray(eid), np.asarray(sid)
  g = np.asarray(gains, np.float32).view(np.uint32).astype(np.uint64)
  per_seg = eid.size // num_sc
  keys, ents = [], []
  for s in range(num_sc):
    start = 0
    for p, end in enumerate(rp[s]):
      end = min(int(end), per_seg)
      for j in range(s * per_seg + start, s * per_seg + max(start, end)):
        if 0 <= eid[j] < rpp and 0 <= sid[j] < bps:
          keys.append(s * bps + sid[j])
          ents.append(np.uint64(p * rpp + eid[j]) | (g[j] << np.uint64(32)))
      start = max(start, (end + 7) // 8 * 8)
  keys = np.asarray(keys, np.int64)
  ents = np.asarray(ents, np.uint64)
  order = np.argsort(keys, kind="stable")
  return keys[order], ents[order]


@pytest.mark.parametrize("num_sc", [1, 4])
def test_sample_stream_is_csr_order_within_rows(num_sc):
  """The CSR-only forward groups the entries by activation row inside the
  call. Its stream must equal a stable sort by row of the CSR's valid
  entries exactly (each row in CSR order, the order in which the oracle
  sums), for rows of 0 to 6000 entries over one and four segments, with
  float gains (weights) so that any order change would also move the
  activations' bits."""
  rng = np.random.default_rng(41 + num_sc)
  vocab = 24000
  sizes = [0, 1, 2, 7, 63, 64, 65, 200, 511, 512, 513, 1000, 4095, 4096, 4097,
           6000, 3, 0, 40, 90]
  batch = len(sizes)
  _, feats = _make_specs(1, [vocab], [8], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch,
                         max_ids=1 << 16)
  embedding.prepare_feature_specs_for_training(feats, 1, num_sc)
  arr = np.empty(batch, dtype=object)
  warr = np.empty(batch, dtype=object)
  for i, n in enumerate(sizes):
    arr[i] = rng.permutation(vocab)[:n].astype(np.int32)
    warr[i] = rng.uniform(0.5, 1.5, size=n).astype(np.float32)
  ref = refcpu.preprocess([arr], [warr], feats, 1, 1,
                          num_sc_per_device=num_sc)
  name = next(iter(ref.row_pointers))
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  bps = batch // num_sc
  keep, c = _device.csr_operands(ref.row_pointers[name],
                                 ref.embedding_ids[name], ref.sample_ids[name],
                                 ref.gains[name], num_sc, num_sc)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  view = _native.build_sample_view(c, batch, rows, device_status=status)
  torch.cuda.synchronize()
  del keep
  assert int(status.item()) == 0
  ek, ee = _expected_sample_stream(ref.row_pointers[name],
                                   ref.embedding_ids[name],
                                   ref.sample_ids[name], ref.gains[name],
                                   num_sc, bps, rows // num_sc)
  gk = view.keys.cpu().numpy().astype(np.int64)
  ge = view.entries.cpu().numpy().view(np.uint64)
  total = ek.size
  np.testing.assert_array_equal(gk[:total], ek)
  np.testing.assert_array_equal(ge[:total], ee)
  assert (gk[total:] == batch).all()
  # The forward through the CSR alone feeds the kernel the same stream.
  table = rng.normal(size=(rows, 8)).astype(np.float32)
  table_t = torch.from_numpy(table).cuda()
  act = _fwd_bind(ref, name, table_t, batch, num_sc).cpu().numpy()
  act_v = _fwd_bind(ref, name, table_t, batch, num_sc,
                    view=view).cpu().numpy()
  np.testing.assert_array_equal(act, act_v)
  args = (ref.row_pointers[name], ref.embedding_ids[name],
          ref.sample_ids[name])
  common = dict(num_sc_per_device=num_sc, num_scs=num_sc)
  exp = refcpu.sparse_dense_matmul(*args, ref.gains[name], table, batch,
                                   **common)
  # Rows of thousands of terms are summed by blocks on the GPU and in one
  # sequence by the oracle: the difference is bounded by a few dozen ulp of
  # the sum of the terms' magnitudes.
  mag = refcpu.sparse_dense_matmul(*args, np.abs(ref.gains[name]),
                                   np.abs(table), batch, **common)
  bound = 32 * np.finfo(np.float32).eps * mag + ATOL
  assert (np.abs(act - exp) <= bound).all()
