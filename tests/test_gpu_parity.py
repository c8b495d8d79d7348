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


@pytest.mark.parametrize("dim", [1, 8, 12, 64, 128, 256, 320])
@pytest.mark.parametrize("num_sc", [1, 4])
def test_forward_matches_oracle(dim, num_sc):
  rng = np.random.default_rng(dim * 7 + num_sc)
  batch = 96
  vocab = 2000
  _, feats = _make_specs(1, [vocab], [dim], "mean",
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  embedding.prepare_feature_specs_for_training(feats, 1, num_sc)
  features = [_ragged(rng, batch, 0, 40, vocab, zipf_a=1.1)]
  name, ref = _csr_from_oracle(features, None, feats, num_sc)
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  table = rng.normal(0, 0.01, size=(rows, dim)).astype(np.float32)
  if dim == 1:
    table = table.reshape(rows)
  act = fwd_prim.tpu_sparse_dense_matmul_csr_primitive.bind(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], 1, torch.from_numpy(table).cuda(),
      device_batch_size=batch, max_ids_per_partition=1 << 20,
      max_unique_ids_per_partition=1 << 20, num_sc_per_device=num_sc)
  exp = refcpu.sparse_dense_matmul(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], table, batch, num_sc_per_device=num_sc, num_scs=num_sc)
  # Sums run in CSR order on both sides: the results agree bit for bit.
  np.testing.assert_array_equal(act.cpu().numpy(), exp)


def _run_grad(optimizer, csr, grad, table0, acc0, lr, lo, hi, num_sc):
  """Runs the GPU primitive and the oracle; returns (got, expected) pairs."""
  table = torch.from_numpy(table0.copy()).cuda()
  if optimizer == "sgd":
    out = sgd_prim.tpu_sparse_dense_matmul_grad_with_sgd_primitive.bind(
        *csr, 1, table, torch.from_numpy(grad).cuda(), lr,
        max_ids_per_partition=1 << 20, max_unique_ids_per_partition=1 << 20,
        min_value=lo, max_value=hi, num_sc_per_device=num_sc)
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
          min_value=lo, max_value=hi, num_sc_per_device=num_sc))
  assert out_t is table and out_a is acc
  exp_t, exp_a = refcpu.sparse_dense_matmul_grad(
      *csr, grad, table0, acc0, learning_rate=lr, num_sc_per_device=num_sc,
      num_scs=num_sc, min_value=lo, max_value=hi)
  return [(table.cpu().numpy(), exp_t), (acc.cpu().numpy(), exp_a)]


@pytest.mark.parametrize("optimizer", ["sgd", "adagrad"])
@pytest.mark.parametrize("dim", [1, 8, 24, 128, 256, 300])
@pytest.mark.parametrize("num_sc", [1, 2])
@pytest.mark.parametrize("clip", [False, True])
def test_grad_hot_rows_exact(optimizer, dim, num_sc, clip):
  """Long runs of hot rows (Zipf 1.05 over 300 rows) cross the backward's
  chunk boundaries and use the multi-piece reduction. Integer-valued
  gradients with unit gains make every partial sum exact, so the result may
  not depend on summation order: GPU and oracle must agree bit for bit."""
  rng = np.random.default_rng(dim * 13 + num_sc + (7 if clip else 0))
  batch = 4096 if dim <= 128 else 512
  vocab = 300
  _, feats = _make_specs(1, [vocab], [dim], "sum",
                         embedding_spec.SGDOptimizerSpec(0.01), batch)
  embedding.prepare_feature_specs_for_training(feats, 1, num_sc)
  features = [_ragged(rng, batch, 1, 8, vocab, zipf_a=1.05)]
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
                            num_sc):
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
                            None, num_sc):
    np.testing.assert_allclose(got, exp, rtol=RTOL, atol=ATOL)


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
