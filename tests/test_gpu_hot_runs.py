"""The backward's hot-run reduction against the oracle.

Long runs of one table row (hot ids) are reduced per sample tile from LDS
instead of one gathered gradient row per entry (segreduce.h, HotPoints ..
HotCombine). By default that happens only when the activation gradients
exceed 16 MB; these cases force it on (SCEMB_HOT_RUNS=1) at sizes the oracle
runs in seconds, check through a profiling span that it ran, and compare:
  * integer-valued gradients with unit gains, where every partial sum is
    exact in any order: bit for bit against the oracle, SGD and Adagrad,
    dims 1 to 300 (the 4- and 16-byte layouts and the column loop);
  * float gradients with weighted gains: bit-identical over repeated calls,
    rows of up to 16 entries against the oracle at the north-star
    tolerance, every row against a float64 restatement within the
    summation bound;
  * the embedding API with Adam and per-feature gradient blocks, against the
    same call with the reduction switched off;
  * hand-made CSRs: runs over the whole batch, with each sample once, or
    three times in one run; a run whose samples are not
    ascending, and one holding a sample id out of range (repeated, unordered
    or bad samples keep a run with the per-entry reduction: exact, the bad
    entry reported as without the hot path); a key order violation next to
    a hot run, still reported; fewer runs taken than found
    (SCEMB_HOT_MAX_RUNS); two partitions; a buffer of padding only.
"""

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


from jax_tpu_embedding.sparsecore import _native  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as adagrad_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd as sgd_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position
from oracle import refcpu  # pylint: disable=g-import-not-at-top,wrong-import-position


@pytest.fixture
def hot(monkeypatch):
  monkeypatch.setenv("SCEMB_HOT_RUNS", "1")
  monkeypatch.delenv("SCEMB_HOT_MAX_RUNS", raising=False)
  return monkeypatch


class _HotLaunches:
  """Counts the hot-run reductions launched inside the block."""

  def __enter__(self):
    _native.profile_enable(True)
    _native.profile_collect(None)
    self.count = 0
    return self

  def __exit__(self, *exc):
    torch.cuda.synchronize()
    self.count = _native.profile_collect("bwd_hot_reduce")[1]
    _native.profile_collect(None)
    _native.profile_enable(False)


def _zipf_rows(rng, batch, lo, hi, vocab, a):
  out = np.empty(batch, dtype=object)
  for i, n in enumerate(rng.integers(lo, hi + 1, size=batch)):
    out[i] = ((rng.zipf(a, size=int(n)) - 1) % vocab).astype(np.int32)
  return out


def _specs(vocab, dim, batch, combiner):
  t = embedding_spec.TableSpec(
      name="t", vocabulary_size=vocab, embedding_dim=dim,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.01), combiner=combiner,
      max_ids_per_partition=1 << 20, max_unique_ids_per_partition=1 << 20)
  feats = [embedding_spec.FeatureSpec(name="f", table_spec=t,
                                      input_shape=[batch, 1],
                                      output_shape=[batch, dim])]
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  return feats


def _entries(rp):
  return int(np.asarray(rp).reshape(-1)[0])


def _grad(optimizer, csr, grad, table0, acc0, lr):
  """GPU primitive (CSR read in place) and oracle: (got, expected) pairs."""
  table = torch.from_numpy(table0.copy()).cuda()
  count = _entries(csr[0])
  kw = dict(max_ids_per_partition=1 << 20,
            max_unique_ids_per_partition=1 << 20, num_sc_per_device=1,
            csr_sorted_by_row=True, csr_num_entries=count)
  if optimizer == "sgd":
    sgd_prim.tpu_sparse_dense_matmul_grad_with_sgd_primitive.bind(
        *csr, 1, table, torch.from_numpy(grad).cuda(), lr, **kw)
    exp_t = refcpu.sparse_dense_matmul_grad(
        *csr, grad, table0, None, learning_rate=lr, num_sc_per_device=1,
        num_scs=1)
    return [(table.cpu().numpy(), exp_t)]
  acc = torch.from_numpy(acc0.copy()).cuda()
  adagrad_prim.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
      *csr, 1, table, acc, torch.from_numpy(grad).cuda(), np.float32(lr),
      **kw)
  exp_t, exp_a = refcpu.sparse_dense_matmul_grad(
      *csr, grad, table0, acc0, learning_rate=lr, num_sc_per_device=1,
      num_scs=1)
  return [(table.cpu().numpy(), exp_t), (acc.cpu().numpy(), exp_a)]


def _oracle_csr(rng, batch, vocab, dim, weighted):
  feats = _specs(vocab, dim, batch, "mean" if weighted else "sum")
  ids = _zipf_rows(rng, batch, 1, 8, vocab, 1.05)
  weights = None
  if weighted:
    weights = np.empty(batch, dtype=object)
    for i, r in enumerate(ids):
      weights[i] = rng.uniform(0.1, 2, size=len(r)).astype(np.float32)
  ref = refcpu.preprocess([ids], None if weights is None else [weights],
                          feats, 1, 1, num_sc_per_device=1)
  name = next(iter(ref.row_pointers))
  csr = (ref.row_pointers[name], ref.embedding_ids[name],
         ref.sample_ids[name], ref.gains[name])
  rows = feats[0].table_spec.stacked_table_spec.stack_vocab_size
  return csr, rows


@pytest.mark.parametrize("optimizer", ["sgd", "adagrad"])
@pytest.mark.parametrize("dim", [1, 8, 24, 128, 300])
def test_hot_runs_exact(hot, optimizer, dim):
  rng = np.random.default_rng(dim * 7 + len(optimizer))
  batch = 4096 if dim <= 128 else 1024
  csr, rows = _oracle_csr(rng, batch, 300, dim, weighted=False)
  assert _entries(csr[0]) > 2 * batch  # the multi-hot kernels
  shape = (rows,) if dim == 1 else (rows, dim)
  table0 = rng.normal(0, 0.01, size=shape).astype(np.float32)
  acc0 = np.full(shape, 0.1, np.float32)
  grad = rng.integers(-3, 4, size=(batch,) if dim == 1 else
                      (batch, dim)).astype(np.float32)
  with _HotLaunches() as h:
    pairs = _grad(optimizer, csr, grad, table0, acc0, 0.05)
  assert h.count == 1
  for got, exp in pairs:
    np.testing.assert_array_equal(got, exp)


def test_hot_runs_float_weighted_deterministic(hot):
  rng = np.random.default_rng(41)
  batch, dim = 4096, 64
  csr, rows = _oracle_csr(rng, batch, 300, dim, weighted=True)
  table0 = rng.normal(0, 0.01, size=(rows, dim)).astype(np.float32)
  acc0 = np.full((rows, dim), 0.1, np.float32)
  grad = rng.normal(0, 1, size=(batch, dim)).astype(np.float32)
  with _HotLaunches() as h:
    runs = [_grad("adagrad", csr, grad, table0, acc0, 0.05) for _ in range(3)]
  assert h.count == 3
  for r in runs[1:]:
    for (got, _), (got0, _) in zip(r, runs[0]):
      np.testing.assert_array_equal(got, got0)
  # Rows of up to 16 entries against the oracle at the north-star tolerance.
  # The hot rows hold thousands: the oracle adds them one after another in
  # fp32, so they are checked against a float64 restatement instead, within
  # the bound of the kernels' summation (chains of at most 84 adds).
  (got_t, exp_t), (got_a, exp_a) = runs[0]
  rp, eid, sid, gains = csr
  n = _entries(rp)
  counts = np.bincount(eid[:n], minlength=rows)
  few = counts <= 16
  np.testing.assert_allclose(got_t[few], exp_t[few], rtol=RTOL, atol=ATOL)
  np.testing.assert_allclose(got_a[few], exp_a[few], rtol=RTOL, atol=ATOL)
  terms = grad[sid[:n]].astype(np.float64) * gains[:n, None].astype(np.float64)
  g64 = np.zeros(table0.shape, np.float64)
  mag = np.zeros(table0.shape, np.float64)
  np.add.at(g64, eid[:n], terms)
  np.add.at(mag, eid[:n], np.abs(terms))
  touched = (counts > 0)[:, None]
  a64 = acc0.astype(np.float64) + np.where(touched, g64 * g64, 0)
  t64 = table0.astype(np.float64) - np.where(
      touched, 0.05 * g64 / np.sqrt(a64), 0)
  e = 5e-6 * mag
  bound_a = 2 * np.abs(g64) * e + e * e + 4e-7 * a64
  bound_t = 0.05 * 0.1**-0.5 * e + 4e-7 * np.abs(t64) + 1e-9
  assert (np.abs(got_a - a64) <= bound_a).all()
  assert (np.abs(got_t - t64) <= bound_t).all()
  assert counts.max() > 500  # runs of more than q = 256 entries are hot


def test_hot_runs_api_adam_row_blocks(monkeypatch):
  """Two features on one table, Adam, per-feature gradient blocks: the same
  update with and without the hot-run reduction."""
  rng = np.random.default_rng(43)
  batch, dim, vocab = 2048, 32, 500
  t = embedding_spec.TableSpec(
      name="t", vocabulary_size=vocab, embedding_dim=dim,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.AdamOptimizerSpec(learning_rate=0.01),
      combiner="sum", max_ids_per_partition=1 << 20,
      max_unique_ids_per_partition=1 << 20)
  feats = [embedding_spec.FeatureSpec(name=f"f{i}", table_spec=t,
                                      input_shape=[batch, 1],
                                      output_shape=[batch, dim])
           for i in range(2)]
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  features = [_zipf_rows(rng, batch, 2, 6, vocab, 1.1) for _ in feats]
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      features, None, feats, 1, 1, num_sc_per_device=1)
  name = feats[0].table_spec.stacked_table_spec.stack_name
  spec = feats[0].table_spec.stacked_table_spec
  shape = (spec.stack_vocab_size, spec.stack_embedding_dim)
  table0 = rng.normal(0, 0.01, size=shape).astype(np.float32)
  grads = [torch.from_numpy(rng.normal(size=(batch, dim)).astype(
      np.float32)).cuda() for _ in feats]
  out = {}
  for mode in ("0", "1"):
    monkeypatch.setenv("SCEMB_HOT_RUNS", mode)
    v = {name: embedding.EmbeddingVariables(
        torch.from_numpy(table0.copy()).cuda(),
        tuple(torch.zeros(shape, dtype=torch.float32, device="cuda")
              for _ in range(2)))}
    with _HotLaunches() as h:
      embedding.tpu_sparse_dense_matmul_grad(
          grads, pre, v, feats, global_device_count=1, num_sc_per_device=1)
    assert h.count == int(mode)
    out[mode] = [v[name].table.cpu().numpy()] + [
        s.cpu().numpy() for s in v[name].slot]
  for a, b in zip(out["1"], out["0"]):
    np.testing.assert_allclose(a, b, rtol=RTOL, atol=ATOL)


def _hand_csr(runs, batch):
  """A one-partition CSR from (row, samples) pairs in the given order."""
  eid = np.concatenate([np.full(len(s), r, np.int32) for r, s in runs])
  sid = np.concatenate([np.asarray(s, np.int32) for _, s in runs])
  n = len(eid)
  rp = np.full(8, n, np.int32)
  return rp, eid, sid, np.ones(n, np.float32)


def _sorted_samples(rng, batch, k):
  return np.sort(rng.choice(batch, size=k, replace=False))


def _integer_case(rng, batch, dim, rows):
  table0 = rng.normal(0, 0.01, size=(rows, dim)).astype(np.float32)
  grad = rng.integers(-3, 4, size=(batch, dim)).astype(np.float32)
  return table0, grad


@pytest.mark.parametrize("copies", [1, 3])
def test_runs_over_the_whole_batch(hot, copies):
  """Every sample in each run: three runs of one entry per sample, or one
  run of three entries per sample (kept with the per-entry reduction)."""
  rng = np.random.default_rng(47)
  batch, dim = 2048, 16
  runs = ([(r, np.arange(batch)) for r in (3, 4, 6)] if copies == 1 else
          [(3, np.repeat(np.arange(batch), copies))])
  csr = _hand_csr(runs, batch)
  assert _entries(csr[0]) > 2 * batch  # the multi-hot kernels
  table0, grad = _integer_case(rng, batch, dim, 8)
  with _HotLaunches() as h:
    (got, exp), = _grad("sgd", csr, grad, table0, None, 0.5)
  assert h.count == 1
  np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("flaw", ["descending", "bad_sample"])
def test_flawed_run_stays_with_per_entry_reduction(hot, flaw):
  rng = np.random.default_rng(53)
  batch, dim = 4096, 8
  good = _sorted_samples(rng, batch, 3000)
  flawed = _sorted_samples(rng, batch, 3000)
  if flaw == "descending":
    flawed[1500], flawed[1501] = flawed[1501], flawed[1500]
  else:
    flawed[1700] = batch + 5
  cold = [(r, _sorted_samples(rng, batch, 40))
          for r in list(range(10, 20)) + list(range(30, 50))]
  runs = [(2, good)] + cold[:10] + [(25, flawed)] + cold[10:] + [(60, good)]
  csr = _hand_csr(runs, batch)
  table0, grad = _integer_case(rng, batch, dim, 64)
  tables = {}
  statuses = {}
  for mode in ("0", "1"):
    hot.setenv("SCEMB_HOT_RUNS", mode)
    keep, c = _device.csr_operands(*csr, 1, 1, sorted_by_row=True,
                                   num_entries=_entries(csr[0]))
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    table = torch.from_numpy(table0.copy()).cuda()
    with _HotLaunches() as h:
      _native.sparse_dense_matmul_grad(c, torch.from_numpy(grad).cuda(),
                                       table, None, 0.5, batch,
                                       device_status=status)
    assert h.count == int(mode)
    del keep
    tables[mode] = table.cpu().numpy()
    statuses[mode] = int(status.item())
  np.testing.assert_array_equal(tables["1"], tables["0"])
  if flaw == "bad_sample":
    assert statuses["1"] == statuses["0"] == _native.STATUS_BAD_ENTRY
  else:
    assert statuses["1"] == statuses["0"] == 0
    exp = refcpu.sparse_dense_matmul_grad(
        *csr, grad, table0, None, learning_rate=0.5, num_sc_per_device=1,
        num_scs=1)
    np.testing.assert_array_equal(tables["1"], exp)


def test_key_order_violation_next_to_hot_run(hot):
  """Row 7 (one entry), then a hot run of row 3, then row 9: SegReduce no
  longer sees 7 next to 3, the hot-run plan must report it."""
  rng = np.random.default_rng(59)
  batch, dim = 2048, 8
  runs = [(7, [5]), (3, _sorted_samples(rng, batch, 2000)),
          (9, _sorted_samples(rng, batch, 1900)),
          (11, _sorted_samples(rng, batch, 300))]
  csr = _hand_csr(runs, batch)
  assert _entries(csr[0]) > 2 * batch  # the multi-hot kernels
  table0, grad = _integer_case(rng, batch, dim, 16)
  keep, c = _device.csr_operands(*csr, 1, 1, sorted_by_row=True,
                                 num_entries=_entries(csr[0]))
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  table = torch.from_numpy(table0.copy()).cuda()
  with _HotLaunches() as h:
    _native.sparse_dense_matmul_grad(c, torch.from_numpy(grad).cuda(), table,
                                     None, 0.5, batch, device_status=status)
  assert h.count == 1
  del keep
  assert int(status.item()) & _native.STATUS_UNSORTED


@pytest.mark.parametrize("max_runs", ["1", "3"])
def test_fewer_runs_taken_than_found(hot, max_runs):
  hot.setenv("SCEMB_HOT_MAX_RUNS", max_runs)
  rng = np.random.default_rng(61)
  batch, dim = 4096, 24
  runs = [(r, _sorted_samples(rng, batch, 1500 + 100 * r)) for r in range(8)]
  csr = _hand_csr(runs, batch)
  table0, grad = _integer_case(rng, batch, dim, 8)
  with _HotLaunches() as h:
    (got, exp), = _grad("sgd", csr, grad, table0, None, 0.25)
  assert h.count == 1
  np.testing.assert_array_equal(got, exp)


def test_two_partitions(hot):
  """Hot runs in both partitions of one segment, with the alignment gap
  between them: keys are partition * rows_per_partition + id."""
  rng = np.random.default_rng(71)
  batch, dim, rpp = 2048, 8, 32
  parts = [[(2, _sorted_samples(rng, batch, 1500)),
            (5, _sorted_samples(rng, batch, 40)),
            (7, _sorted_samples(rng, batch, 1500))],
           [(1, _sorted_samples(rng, batch, 1500)),
            (9, _sorted_samples(rng, batch, 1200))]]
  eid, sid, rp = [], [], []
  for runs in parts:
    start = (len(eid) + 7) // 8 * 8
    pad = start - len(eid)
    eid += [np.iinfo(np.int32).max] * pad
    sid += [np.iinfo(np.int32).max] * pad
    for r, samples in runs:
      eid += [r] * len(samples)
      sid += list(samples)
    rp.append(len(eid))
  rp = np.array(rp + [rp[-1]] * (8 - len(rp)), np.int32)
  eid = np.array(eid, np.int32)
  sid = np.array(sid, np.int32)
  gains = np.ones(len(eid), np.float32)
  assert len(eid) > 2 * batch  # the multi-hot kernels
  table0, grad = _integer_case(rng, batch, dim, 2 * rpp)
  keep, c = _device.csr_operands(rp, eid, sid, gains, 1, 2,
                                 sorted_by_row=True, num_entries=len(eid))
  table = torch.from_numpy(table0.copy()).cuda()
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  with _HotLaunches() as h:
    _native.sparse_dense_matmul_grad(c, torch.from_numpy(grad).cuda(), table,
                                     None, 0.5, batch, device_status=status)
  assert h.count == 1
  del keep
  assert int(status.item()) == 0
  exp = refcpu.sparse_dense_matmul_grad(
      rp, eid, sid, gains, grad, table0, None, learning_rate=0.5,
      num_sc_per_device=1, num_scs=2)
  np.testing.assert_array_equal(table.cpu().numpy(), exp)


def test_padding_only(hot):
  """A buffer of 3 * batch positions whose partition holds no entry."""
  rng = np.random.default_rng(67)
  batch, dim = 1024, 8
  n = 3 * batch
  rp = np.zeros(8, np.int32)
  eid = np.full(n, np.iinfo(np.int32).max, np.int32)
  sid = np.full(n, np.iinfo(np.int32).max, np.int32)
  gains = np.full(n, np.nan, np.float32)
  table0, grad = _integer_case(rng, batch, dim, 16)
  keep, c = _device.csr_operands(rp, eid, sid, gains, 1, 1,
                                 sorted_by_row=True, num_entries=n)
  table = torch.from_numpy(table0.copy()).cuda()
  with _HotLaunches() as h:
    _native.sparse_dense_matmul_grad(c, torch.from_numpy(grad).cuda(), table,
                                     None, 0.5, batch)
  assert h.count == 1
  del keep
  np.testing.assert_array_equal(table.cpu().numpy(), table0)
