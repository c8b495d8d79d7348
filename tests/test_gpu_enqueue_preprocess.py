"""Preprocessing enqueued without the wait for its stats
(embedding.enqueue_preprocess_sparse_dense_matmul_input): the same buffers
and stats as the synchronous entry, usable by work enqueued after it, in a
training loop that preprocesses batch k + 1 on a side stream during step k,
and with the same errors, raised by result()."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  torch.cuda.set_device(0)


from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position


def _specs(batch, limit=1 << 20, dims=(16, 16, 32)):
  tables = [embedding_spec.TableSpec(
      name=f"t{i}", vocabulary_size=int(v), embedding_dim=d,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner="mean",
      max_ids_per_partition=limit, max_unique_ids_per_partition=limit)
            for i, (v, d) in enumerate(zip((300, 9000, 40), dims))]
  feats = [embedding_spec.FeatureSpec(
      name=f"f{i}", table_spec=t, input_shape=[batch, 1],
      output_shape=[batch, t.embedding_dim]) for i, t in enumerate(tables)]
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  return feats


def _batch(rng, feats):
  out = []
  for fs in feats:
    v, b = fs.table_spec.vocabulary_size, fs.input_shape[0]
    rows = np.empty(b, dtype=object)
    for i in range(b):
      rows[i] = rng.integers(0, v, size=int(rng.integers(0, 12))).astype(
          np.int32)
    out.append(rows)
  return out


def _written(pre):
  """Row pointers and the written entries of every stack (the buffers past
  the row pointers' end are not written)."""
  out = {}
  for name, rp in pre.lhs_row_pointers.items():
    rp = rp.cpu().numpy()
    n = int(rp[-1])
    out[name] = [rp] + [
        x[name].cpu().numpy().view(np.int32)[:n]
        for x in (pre.lhs_embedding_ids, pre.lhs_sample_ids, pre.lhs_gains)]
  return out


def _same(a, b):
  assert a.keys() == b.keys()
  for k in a:
    for x, y in zip(a[k], b[k]):
      np.testing.assert_array_equal(x, y)


def _same_stats(s, t):
  for f in ("max_ids_per_partition", "max_unique_ids_per_partition",
            "required_buffer_size_per_sc", "id_drop_counters"):
    a, b = getattr(s, f), getattr(t, f)
    assert a.keys() == b.keys()
    for k in a:
      np.testing.assert_array_equal(a[k], b[k])


def test_enqueue_matches_synchronous_entry():
  rng = np.random.default_rng(1)
  feats = _specs(256)
  ids = _batch(rng, feats)
  pre_s, stats_s = embedding.preprocess_sparse_dense_matmul_input(
      ids, None, feats, 1, 1, num_sc_per_device=1)
  pre_a, pending = embedding.enqueue_preprocess_sparse_dense_matmul_input(
      ids, None, feats, 1, 1, num_sc_per_device=1)
  assert pre_a.csr_num_entries is None  # known once the stats are in
  stats_a = pending.result()
  assert pending.result() is stats_a
  _same(_written(pre_s), _written(pre_a))
  _same_stats(stats_s, stats_a)
  assert pre_a.csr_num_entries == pre_s.csr_num_entries
  for name, view in pre_a.lookup_views.items():
    assert view.num_entries == pre_s.lookup_views[name].num_entries
    np.testing.assert_array_equal(view.keys.cpu().numpy(),
                                  pre_s.lookup_views[name].keys.cpu().numpy())


def test_pipelined_loop_on_a_side_stream():
  """Batch k + 1 preprocessed on a side stream while step k (a lookup of
  batch k) runs; each batch's activations equal those of the synchronous
  entry, and result() comes after the next step is enqueued."""
  rng = np.random.default_rng(2)
  feats = _specs(512)
  batches = [_batch(rng, feats) for _ in range(5)]
  tables = {}
  for name, spec in embedding.get_stacked_table_specs(feats).items():
    tables[name] = embedding.EmbeddingVariables(
        table=torch.tensor(rng.normal(size=(
            spec.stack_vocab_size, spec.stack_embedding_dim)).astype(
                np.float32)).cuda(), slot=())
  expected = []
  for ids in batches:
    pre, _ = embedding.preprocess_sparse_dense_matmul_input(
        ids, None, feats, 1, 1, num_sc_per_device=1)
    acts = embedding.tpu_sparse_dense_matmul(pre, tables, feats,
                                             global_device_count=1)
    expected.append([a.cpu().numpy() for a in acts])
  main = torch.cuda.current_stream()
  side = torch.cuda.Stream()

  def enqueue(ids):
    with torch.cuda.stream(side):
      pre, stats = embedding.enqueue_preprocess_sparse_dense_matmul_input(
          ids, None, feats, 1, 1, num_sc_per_device=1)
    main.wait_stream(side)
    return pre, stats

  got = []
  cur, stats = enqueue(batches[0])
  for k in range(len(batches)):
    acts = embedding.tpu_sparse_dense_matmul(cur, tables, feats,
                                             global_device_count=1)
    nxt = enqueue(batches[k + 1]) if k + 1 < len(batches) else None
    stats.result()
    got.append(acts)
    if nxt is not None:
      cur, stats = nxt
  torch.cuda.synchronize()
  for g, e in zip(got, expected):
    for a, b in zip(g, e):
      np.testing.assert_array_equal(a.cpu().numpy(), b)


def test_result_raises_like_the_synchronous_entry():
  rng = np.random.default_rng(3)
  feats = _specs(256, limit=2)
  ids = _batch(rng, feats)
  _, pending = embedding.enqueue_preprocess_sparse_dense_matmul_input(
      ids, None, feats, 1, 1, num_sc_per_device=1)
  with pytest.raises(RuntimeError, match="max ids per partition"):
    pending.result()
  bad = _batch(rng, _specs(256))
  bad[0][3] = np.array([-5], np.int32)
  _, pending = embedding.enqueue_preprocess_sparse_dense_matmul_input(
      bad, None, _specs(256), 1, 1, num_sc_per_device=1)
  with pytest.raises(ValueError, match="negative or beyond"):
    pending.result()
