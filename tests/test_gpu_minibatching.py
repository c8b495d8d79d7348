"""GPU parity of minibatching (enable_minibatching, single host).

* Preprocessing: every pass against the CPU oracle, bit for bit on the
  written region of the CSR (row pointers of all minibatches, entries and
  alignment padding up to the last row pointer), plus the minibatch count,
  the stats (first pass) and the dropped ids (last pass). The minibatch
  contents depend on the HighwayHash bucket of every column id, so these also
  pin the device hash.
* Lookup and update over the minibatched CSR: against the oracle reading the
  same layout (rtol 1e-5, atol 1e-6, the fp32 tolerance of the other parity
  tests), and against the CSR built without minibatching.
* The reference's own minibatching tests: the two-minibatch forward and SGD
  cases of primitives/tests/sparse_dense_matmul_csr_minibatching_test.py:
  399-591 and sparse_dense_matmul_grad_with_sgd_minibatching_test.py:161-275
  (explicit minibatches through lib/core/input_preprocessing), and the
  single-host cases of lib/nn/tests/minibatching_test.py:192-398.
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


from jax_tpu_embedding.sparsecore.lib.core import input_preprocessing  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr as fwd_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as adagrad_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd as sgd_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.utils import utils  # pylint: disable=g-import-not-at-top,wrong-import-position
from oracle import refcpu  # pylint: disable=g-import-not-at-top,wrong-import-position


def _specs(tables, batch, limits, num_sc, combiner="sum", devices=1):
  """One feature per (name, vocab, dim) table, stacked by dimension."""
  specs = []
  for name, vocab, dim in tables:
    t = embedding_spec.TableSpec(
        name=name, vocabulary_size=vocab, embedding_dim=dim,
        initializer=embedding_spec.zeros,
        optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner=combiner,
        max_ids_per_partition=limits[0],
        max_unique_ids_per_partition=limits[1])
    specs.append(embedding_spec.FeatureSpec(
        name=f"f_{name}", table_spec=t, input_shape=[batch, 1],
        output_shape=[batch, dim]))
  embedding.prepare_feature_specs_for_training(specs, devices, num_sc)
  return specs


def _ragged(rng, batch, lo, hi, vocab):
  arr = np.empty(batch, dtype=object)
  for i in range(batch):
    arr[i] = rng.integers(0, vocab, size=int(rng.integers(lo, hi + 1))
                          ).astype(np.int32)
  return arr


def _weights_like(rng, ragged):
  arr = np.empty(len(ragged), dtype=object)
  for i, r in enumerate(ragged):
    arr[i] = rng.uniform(0.1, 1, size=len(r)).astype(np.float32)
  return arr


def _written_end(rp, nmb, num_sc, rpb):
  """Aligned end of the last minibatch's last partition of a device."""
  block = rp[:num_sc * nmb * rpb]
  return int(-(-int(block.max()) // 8) * 8) if block.size else 0


def _compare(features, weights, specs, num_sc, *, allow, L=1, G=1):
  got = pip.preprocess_sparse_dense_matmul_input(
      features, weights, specs, L, G, num_sc_per_device=num_sc,
      allow_id_dropping=allow, enable_minibatching=True)
  rps, eids, sids, gns, nmb, stats = got
  ref = refcpu.preprocess(features, weights, specs, L, G,
                          num_sc_per_device=num_sc, allow_id_dropping=allow,
                          enable_minibatching=True)
  assert nmb == ref.num_minibatches
  ns = num_sc * G
  rpb = max(ns, 8)
  for name in ref.row_pointers:
    rp_all = rps[name].cpu().numpy()
    assert rp_all.size == L * num_sc * 64 * rpb
    c = eids[name].numel() // L
    for d in range(L):
      rp = rp_all[d * num_sc * 64 * rpb:(d + 1) * num_sc * 64 * rpb]
      rp_ref = ref.row_pointers[name][d * num_sc * 64 * rpb:]
      n_rp = num_sc * nmb * rpb
      np.testing.assert_array_equal(rp[:n_rp], rp_ref[:n_rp], err_msg=name)
      end = min(_written_end(rp, nmb, num_sc, rpb), c)
      for got_d, exp_d in ((eids, ref.embedding_ids), (sids, ref.sample_ids),
                           (gns, ref.gains)):
        g = got_d[name].cpu().numpy()[d * c:d * c + end]
        e = exp_d[name][d * c:d * c + end]
        np.testing.assert_array_equal(g.view(np.int32), e.view(np.int32),
                                      err_msg=f"{name} device {d}")
    np.testing.assert_array_equal(stats.max_ids_per_partition[name],
                                  ref.max_ids_per_partition[name])
    np.testing.assert_array_equal(stats.max_unique_ids_per_partition[name],
                                  ref.max_unique_ids_per_partition[name])
    np.testing.assert_array_equal(stats.required_buffer_sizes[name],
                                  ref.required_buffer_sizes[name])
    assert stats.dropped_id_count[name] == ref.dropped_id_count[name], name
  return got, ref


@pytest.mark.parametrize("num_sc", [1, 2, 4])
def test_not_required_keeps_one_minibatch(num_sc):
  """Limits that hold: one minibatch, in the minibatching layout (device
  positions, SCs packed by their required sizes)."""
  rng = np.random.default_rng(num_sc)
  specs = _specs([("a", 4096, 16), ("b", 1000, 16)], 64, (1 << 16, 1 << 16),
                 num_sc)
  feats = [_ragged(rng, 64, 0, 9, 4096), _ragged(rng, 64, 1, 4, 1000)]
  (_, _, _, _, nmb, _), _ = _compare(feats, None, specs, num_sc, allow=False)
  assert nmb == 1


@pytest.mark.parametrize("num_sc,combiner,weighted,limits", [
    (1, "sum", False, (8, 6)),
    (1, "mean", True, (5, 5)),
    (2, "sqrtn", False, (6, 3)),
    (4, "sum", True, (4, 4)),
    (4, "mean", False, (2, 2)),
    (2, "sum", False, (1, 1)),
])
def test_required_matches_oracle(num_sc, combiner, weighted, limits):
  """Two stacks (different dims) whose splits OR together; ids dropped per
  (partition, bucket)."""
  rng = np.random.default_rng(hash((num_sc, combiner, weighted)) % 2**32)
  batch = 128
  specs = _specs([("a", 6000, 8), ("b", 900, 16), ("c", 3000, 16)], batch,
                 limits, num_sc, combiner)
  feats = [_ragged(rng, batch, 0, 12, 6000), _ragged(rng, batch, 1, 5, 900),
           _ragged(rng, batch, 0, 3, 3000)]
  weights = [_weights_like(rng, f) for f in feats] if weighted else None
  (_, _, _, _, nmb, _), _ = _compare(feats, weights, specs, num_sc,
                                     allow=True)
  assert nmb > 1


def test_required_without_dropping_raises():
  """A bucket over a limit with dropping off: RuntimeError (the reference
  LOG(FATAL)s, sort_and_group_coo_tensors_impl.h:564-570)."""
  rng = np.random.default_rng(5)
  specs = _specs([("a", 64, 8)], 64, (2, 2), 1)
  feats = [_ragged(rng, 64, 4, 8, 64)]
  with pytest.raises(RuntimeError):
    pip.preprocess_sparse_dense_matmul_input(
        feats, None, specs, 1, 1, num_sc_per_device=1,
        allow_id_dropping=False, enable_minibatching=True)
  with pytest.raises(RuntimeError):
    refcpu.preprocess(feats, None, specs, 1, 1, num_sc_per_device=1,
                      allow_id_dropping=False, enable_minibatching=True)


def test_two_local_devices():
  rng = np.random.default_rng(11)
  specs = _specs([("a", 8000, 8)], 128, (3, 3), 2, devices=2)
  feats = [_ragged(rng, 128, 0, 6, 8000)]
  _compare(feats, None, specs, 2, allow=True, L=2, G=2)


def test_small_buffer_drops_like_the_oracle():
  """A suggested buffer too small for the minibatches: the static-buffer
  drops of FillBufferSegment (input_preprocessing_util.cc:73-95)."""
  rng = np.random.default_rng(3)
  specs = _specs([("a", 4000, 8)], 256, (3, 3), 2)
  specs[0].table_spec.stacked_table_spec = (
      specs[0].table_spec.stacked_table_spec.replace(
          suggested_coo_buffer_size_per_device=64))
  feats = [_ragged(rng, 256, 1, 6, 4000)]
  (_, _, _, _, _, stats), ref = _compare(feats, None, specs, 2, allow=True)
  name = specs[0].table_spec.stacked_table_spec.stack_name
  assert stats.dropped_id_count[name] > 0


def _csr_args(got, name):
  rps, eids, sids, gns, nmb, _ = got
  return (rps[name], eids[name], sids[name], gns[name]), nmb


@pytest.mark.parametrize("num_sc,dim", [(1, 16), (4, 8), (2, 128)])
def test_lookup_and_update_over_minibatches(num_sc, dim):
  rng = np.random.default_rng(dim + num_sc)
  batch, vocab = 256, 2048
  specs = _specs([("a", vocab, dim)], batch, (3, 3), num_sc)
  feats = [_ragged(rng, batch, 1, 8, vocab)]
  got, ref = _compare(feats, None, specs, num_sc, allow=True)
  name = specs[0].table_spec.stacked_table_spec.stack_name
  (rp, eid, sid, gains), nmb = _csr_args(got, name)
  assert nmb > 1
  table = rng.normal(size=(vocab, dim)).astype(np.float32)
  kw = dict(device_batch_size=batch, max_ids_per_partition=3,
            max_unique_ids_per_partition=3, num_sc_per_device=num_sc,
            global_device_count=1, enable_minibatching=True)
  act = fwd_prim.tpu_sparse_dense_matmul_csr_primitive.bind(
      rp, eid, sid, gains, np.int32(nmb), torch.tensor(table).cuda(), **kw)
  exp = refcpu.sparse_dense_matmul(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], table, batch, num_sc_per_device=num_sc,
      num_scs=num_sc, num_minibatches=nmb)
  np.testing.assert_allclose(act.cpu().numpy(), exp, rtol=RTOL, atol=ATOL)
  grad = rng.normal(size=(batch, dim)).astype(np.float32)
  tab = torch.tensor(table).cuda()
  acc = torch.full((vocab, dim), 0.1, device="cuda")
  adagrad_prim.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
      rp, eid, sid, gains, np.int32(nmb), tab, acc, torch.tensor(grad).cuda(),
      0.05, max_ids_per_partition=3, max_unique_ids_per_partition=3,
      computation_name="adagrad", num_sc_per_device=num_sc,
      global_device_count=1, enable_minibatching=True,
      csr_sorted_by_row=True)
  exp_t, exp_a = refcpu.sparse_dense_matmul_grad(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], grad, table, np.full((vocab, dim), 0.1, np.float32),
      learning_rate=0.05, num_sc_per_device=num_sc, num_scs=num_sc,
      num_minibatches=nmb)
  np.testing.assert_allclose(tab.cpu().numpy(), exp_t, rtol=RTOL, atol=ATOL)
  np.testing.assert_allclose(acc.cpu().numpy(), exp_a, rtol=RTOL, atol=ATOL)


def test_entry_bound_skips_the_unused_buffer():
  """The buffer is sized for 64 minibatches; with the preprocessing's entry
  count the lookup and update only visit the positions the minibatches can
  use. Same results, bit for bit, as over the whole buffer."""
  rng = np.random.default_rng(17)
  batch, vocab, dim, limit = 4096, 50000, 16, 4096
  specs = _specs([("a", vocab, dim)], batch, (limit, limit), 1)
  feats = [_ragged(rng, batch, 1, 8, vocab)]
  got, _ = _compare(feats, None, specs, 1, allow=False)
  name = specs[0].table_spec.stacked_table_spec.stack_name
  (rp, eid, sid, gains), nmb = _csr_args(got, name)
  entries = got[5].num_entries[name]
  assert nmb > 1 and 0 < 8 * entries < eid.numel()
  table = rng.normal(size=(vocab, dim)).astype(np.float32)
  grad = torch.tensor(rng.normal(size=(batch, dim)).astype(np.float32)).cuda()
  kw = dict(max_ids_per_partition=limit, max_unique_ids_per_partition=limit,
            num_sc_per_device=1, global_device_count=1,
            enable_minibatching=True)
  outs = []
  # Whole buffer, sorted backward; bounded, sorted (the same sorted stream:
  # equal bit for bit); bounded, the CSR read in place (one SparseCore: every
  # row's entries are contiguous; a row is summed in the same order but split
  # into pieces at other positions, so to rounding).
  for n, in_place in ((None, False), (entries, False), (entries, True)):
    act = fwd_prim.tpu_sparse_dense_matmul_csr_primitive.bind(
        rp, eid, sid, gains, nmb, torch.tensor(table).cuda(),
        device_batch_size=batch, csr_num_entries=n, **kw)
    tab = torch.tensor(table).cuda()
    acc = torch.full((vocab, dim), 0.1, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    adagrad_prim.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
        rp, eid, sid, gains, nmb, tab, acc, grad, 0.05,
        computation_name="adagrad", csr_num_entries=n,
        csr_sorted_by_row=in_place, **kw)
    outs.append([x.cpu().numpy() for x in (act, tab, acc)])
  for a, b in zip(outs[0], outs[1]):
    np.testing.assert_array_equal(a, b)
  for a, b in zip(outs[0], outs[2]):
    np.testing.assert_allclose(a, b, rtol=RTOL, atol=ATOL)
  del status


# ---------------------------------------------------------------------------
# The reference's minibatching tests.
# ---------------------------------------------------------------------------

# sparse_dense_matmul_csr_minibatching_test.py:403-423 (and the SGD test's
# identical inputs).
_MB0 = [[5], [3], [], [1], [6], [], [0], [4], [], [], [], [7], [], [], [2], []]
_MB1 = [[], [], [9], [], [], [12], [], [], [15], [13], [11], [], [8], [14], [],
        [10]]


def _explicit_minibatches():
  mb0, mb1 = _MB0 * 2, _MB1 * 2
  w0 = [[1.0] * len(r) for r in mb0]
  w1 = [[1.0] * len(r) for r in mb1]
  return [mb0, mb1], [w0, w1]


@pytest.mark.parametrize("num_sc", [1, 2, 4])
def test_reference_forward_two_minibatches_per_core(num_sc):
  """Row i of the table holds i; each sample's activation is its id
  (csr_minibatching_test.py:399-495, :497-591)."""
  vocab, dim, batch = 32, 8, 32
  features, weights = _explicit_minibatches()
  rp, eid, sid, gains = input_preprocessing.preprocess_sparse_dense_matmul_input(
      features, weights, 1, num_sc_per_device=num_sc,
      max_ids_per_partition=16, max_unique_ids_per_partition=16,
      enable_minibatching=True)
  table = np.tile(np.arange(vocab, dtype=np.float32)[:, None], (1, dim))
  sharded = utils.shard_emb_table(table, num_devices=1,
                                  num_sc_per_device=num_sc)[0]
  act = fwd_prim.tpu_sparse_dense_matmul_csr_primitive.bind(
      rp, eid, sid, gains, 2, torch.tensor(np.ascontiguousarray(sharded)).cuda(),
      device_batch_size=batch, max_ids_per_partition=16,
      max_unique_ids_per_partition=16, sharding_strategy=1,
      enable_minibatching=True, num_sc_per_device=num_sc,
      global_device_count=1)
  ids = [(a or b)[0] for a, b in zip(features[0], features[1])]
  expected = np.tile(np.array(ids, np.float32)[:, None], (1, dim))
  np.testing.assert_array_equal(act.cpu().numpy(), expected)


@pytest.mark.parametrize("num_sc", [1, 4])
@pytest.mark.parametrize("clip", [None, (2.0, 12.0)])
def test_reference_sgd_two_minibatches_per_core(num_sc, clip):
  """Rows 0-15 each get two unit gradients: -0.2 at learning rate 0.1, then
  the clip (sgd_minibatching_test.py:161-275)."""
  vocab, dim, batch = 32, 8, 32
  features, weights = _explicit_minibatches()
  rp, eid, sid, gains = input_preprocessing.preprocess_sparse_dense_matmul_input(
      features, weights, 1, num_sc_per_device=num_sc,
      max_ids_per_partition=16, max_unique_ids_per_partition=16,
      enable_minibatching=True)
  table = np.tile(np.arange(vocab, dtype=np.float32)[:, None], (1, dim))
  sharded = torch.tensor(np.ascontiguousarray(utils.shard_emb_table(
      table, num_devices=1, num_sc_per_device=num_sc)[0])).cuda()
  lo, hi = clip if clip else (None, None)
  out = sgd_prim.tpu_sparse_dense_matmul_grad_with_sgd_primitive.bind(
      rp, eid, sid, gains, 2, sharded, torch.ones(batch, dim).cuda(), 0.1,
      max_ids_per_partition=16, max_unique_ids_per_partition=16,
      computation_name="sgd_test_computation", sharding_strategy=1,
      enable_minibatching=True, min_value=lo, max_value=hi,
      num_sc_per_device=num_sc, global_device_count=1)
  got = utils.unshard_emb_table(out.cpu().numpy()[None], num_sc_per_device=num_sc)
  expected = table.copy()
  updated = np.unique(np.concatenate([np.array(r, int) for mb in features
                                      for r in mb if r]))
  expected[updated, :] -= 0.2
  if clip:
    expected[updated, :] = np.clip(expected[updated, :], lo, hi)
  np.testing.assert_allclose(got, expected, atol=1e-5)


def _nn_case(limits, batch=16, max_sample=20, seed=2025, allow=True):
  """lib/nn/tests/minibatching_test.py:126-189: one 2048 x 16 SGD table."""
  num_sc = utils.num_sparsecores_per_device()
  table = embedding_spec.TableSpec(
      vocabulary_size=2048, embedding_dim=16,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(), combiner="sum",
      name="table_a")
  feature = embedding_spec.FeatureSpec(
      table_spec=table, input_shape=[batch, 1], output_shape=[batch, 16],
      name="feature_a")
  embedding.prepare_feature_specs_for_training([feature], 1, num_sc)
  st = feature.table_spec.stacked_table_spec
  feature.table_spec.stacked_table_spec = st.replace(
      max_ids_per_partition=limits[0], max_unique_ids_per_partition=limits[1])
  rng = np.random.RandomState(seed)
  inputs = np.empty(batch, dtype=object)
  for i in range(batch):
    inputs[i] = rng.randint(0, 2048, size=(rng.randint(1, max_sample + 1),),
                            dtype=np.int32)
  pre, stats = embedding.preprocess_sparse_dense_matmul_input(
      [inputs], None, [feature], 1, 1, num_sc_per_device=num_sc,
      batch_number=42, enable_minibatching=True, allow_id_dropping=allow)
  return feature, inputs, pre, stats, num_sc


def test_nn_not_required_and_required_counts():
  """minibatching_test.py:192-225."""
  _, _, pre, _, _ = _nn_case((1 << 16, 1 << 16), max_sample=8)
  assert (pre.num_minibatches == 1).all()
  _, _, pre, _, _ = _nn_case((1, 1))
  assert (pre.num_minibatches > 1).all()


def test_nn_id_dropping_counted():
  """minibatching_test.py:227-303: ids and unique ids over the per-bucket
  limits are dropped and counted."""
  for limits in ((1, 1), (10, 1)):
    _, _, _, stats, _ = _nn_case(limits, batch=64, max_sample=8)
    assert stats.id_drop_counters["table_a"] > 0


def test_nn_views_and_in_place_backward_match_the_plain_csr():
  """Through the embedding API the minibatched step takes the sample view
  built by the final pass (trimmed to the entries) and the in-place
  backward; the same CSR without them (sorting in every call) gives the same
  tables and activations (rtol 1e-5: the view orders a row's entries by
  input position, the sorted CSR by column; the in-place backward splits a
  row's sum at other positions)."""
  feature, _, pre, _, num_sc = _nn_case((64, 64), batch=64)
  assert (pre.num_minibatches > 1).all()
  name = feature.table_spec.stacked_table_spec.stack_name
  view = pre.lookup_views[name]
  assert view is not None and view.keys.numel() < (
      pre.sparse_dense_matmul_input.lhs_embedding_ids[name].numel())
  rng = np.random.default_rng(2)
  table = rng.normal(size=(2048, 16)).astype(np.float32)
  grads = torch.tensor(rng.normal(size=(64, 16)).astype(np.float32)).cuda()
  results = []
  for plain in (False, True):
    p = pre
    if plain:
      p = embedding.PreprocessedInput(pre.sparse_dense_matmul_input,
                                      pre.num_minibatches)
    variables = {name: embedding.EmbeddingVariables(
        table=torch.tensor(table).cuda(), slot=())}
    acts = embedding.tpu_sparse_dense_matmul(
        p, variables, [feature], global_device_count=1,
        num_sc_per_device=num_sc, enable_minibatching=True)
    upd = embedding.tpu_sparse_dense_matmul_grad(
        [grads], p, variables, [feature], num_sc_per_device=num_sc,
        enable_minibatching=True)
    results.append((acts[0].cpu().numpy(), upd[name].table.cpu().numpy()))
  for a, b in zip(results[0], results[1]):
    np.testing.assert_allclose(a, b, rtol=RTOL, atol=ATOL)


def test_nn_forward_and_backward():
  """minibatching_test.py:322-398: a row-initialised table looks up the sum
  of each sample's ids; SGD with unit gradients lowers each row by the
  learning rate times its count. With one SparseCore the reference's limit
  of 2 ids per partition drops ids, so the limits here are 8 (several
  minibatches, nothing dropped)."""
  feature, inputs, pre, stats, num_sc = _nn_case((8, 8))
  assert (pre.num_minibatches > 1).all()
  assert stats.id_drop_counters["table_a"] == 0
  vocab, dim = 2048, 16
  logical = np.tile(np.arange(vocab, dtype=np.float32)[:, None], (1, dim))
  sharded = torch.tensor(np.ascontiguousarray(utils.shard_emb_table(
      logical, num_devices=1, num_sc_per_device=num_sc)[0])).cuda()
  variables = {"table_a": embedding.EmbeddingVariables(table=sharded, slot=())}
  acts = embedding.tpu_sparse_dense_matmul(
      pre, variables, [feature], global_device_count=1,
      num_sc_per_device=num_sc, enable_minibatching=True)
  expected = np.tile(np.array([r.sum() for r in inputs], np.float32)[:, None],
                     (1, dim))
  np.testing.assert_allclose(acts[0].cpu().numpy(), expected, rtol=1e-6)
  updated = embedding.tpu_sparse_dense_matmul_grad(
      [torch.ones(16, dim).cuda()], pre, variables, [feature],
      num_sc_per_device=num_sc, enable_minibatching=True)
  counts = np.bincount(np.concatenate(list(inputs)), minlength=vocab)
  lr = np.float32(feature.table_spec.optimizer.learning_rate)
  exp_logical = logical - lr * counts[:, None].astype(np.float32)
  got = utils.unshard_emb_table(updated["table_a"].table.cpu().numpy()[None],
                                num_sc_per_device=num_sc)
  np.testing.assert_allclose(got, exp_logical, rtol=1e-6)


@pytest.mark.parametrize("num_sc,limits,weighted", [
    (1, (8, 6), False), (2, (3, 3), True), (4, (2, 1), False),
    (1, (1, 1), True)])
def test_first_pass_split_equals_bucket_pass_split(num_sc, limits, weighted):
  """The split the first pass counts from its runs is the bucket pass's
  (library pass 1), stack by stack; the split decides the whole minibatched
  CSR, which the other tests compare with the oracle."""
  rng = np.random.default_rng(num_sc * 7 + limits[0])
  batch = 256
  specs = _specs([("a", 3000, 8), ("b", 500, 16)], batch, limits, num_sc)
  feats = [_ragged(rng, batch, 0, 9, 3000), _ragged(rng, batch, 1, 4, 500)]
  weights = [_weights_like(rng, f) for f in feats] if weighted else None
  stacks = pip.get_stacked_table_metadata(specs)
  for name, metas in stacks.items():
    dev = [pip._to_device_feature(feats[m.feature_index],  # pylint: disable=protected-access
                                  None if weights is None else
                                  weights[m.feature_index]) for m in metas]
    kw = dict(feats=dev, metas=metas, local_device_count=1,
              global_device_count=1, num_sc_per_device=num_sc,
              allow_id_dropping=True, has_weights=weighted,
              enable_minibatching=True)
    first = pip._preprocess_stack(**kw, minibatching_pass=0)  # pylint: disable=protected-access
    bucket = pip._preprocess_stack(**kw, minibatching_pass=1,  # pylint: disable=protected-access
                                   outputs=first[:4])
    c0, c1 = pip._read_counters([(first[4], first[5][3]),  # pylint: disable=protected-access
                                 (bucket[4], bucket[5][3])])
    assert c0[4] == 1, name
    assert c0[5] == c1[5] and c1[5] != 0, name
