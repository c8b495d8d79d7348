"""Randomised GPU-vs-oracle parity over the option space.

Each case draws SparseCores per device (1, 2, 4), one or two devices (local
or global), combiner, weights, id dropping, minibatching, the id limits and
one to three tables, then checks:
- preprocessing bit for bit (row pointers, entries on the compared region,
  stats, dropped ids), or that GPU and oracle both raise (limits exceeded
  with dropping off);
- on one device, the lookup and Adagrad over the produced CSR against the
  oracle at rtol 1e-5 / atol 1e-6.
"""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  torch.cuda.set_device(0)


from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr as fwd_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as ada_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position
from oracle import refcpu  # pylint: disable=g-import-not-at-top,wrong-import-position

RTOL, ATOL = 1e-5, 1e-6
CASES_PER_TEST = 25


def _specs(tables, batch, limits, num_sc, combiner, devices):
  specs = []
  for name, vocab, dim in tables:
    t = embedding_spec.TableSpec(
        name=name, vocabulary_size=vocab, embedding_dim=dim,
        initializer=embedding_spec.zeros,
        optimizer=embedding_spec.AdagradOptimizerSpec(0.05), combiner=combiner,
        max_ids_per_partition=limits[0],
        max_unique_ids_per_partition=limits[1])
    specs.append(embedding_spec.FeatureSpec(
        name=f"f_{name}", table_spec=t, input_shape=[batch, 1],
        output_shape=[batch, dim]))
  embedding.prepare_feature_specs_for_training(specs, devices, num_sc)
  return specs


def _ragged(rng, batch, hi, vocab):
  arr = np.empty(batch, dtype=object)
  for i in range(batch):
    arr[i] = rng.integers(0, vocab, size=int(rng.integers(0, hi + 1))
                          ).astype(np.int32)
  return arr


def _draw(seed):
  rng = np.random.default_rng(seed)
  c = dict(S=int(rng.choice([1, 2, 4])), G=int(rng.choice([1, 1, 2])))
  c["L"] = int(rng.choice([1, c["G"]]))
  c["combiner"] = str(rng.choice(["sum", "mean", "sqrtn"]))
  c["weighted"] = bool(rng.integers(0, 2))
  c["mb"] = bool(rng.integers(0, 2))
  c["allow"] = bool(rng.integers(0, 2)) or c["mb"]
  batch = int(rng.choice([64, 128, 256])) * c["G"]
  tables = [(f"t{i}", int(rng.integers(50, 5000)), int(rng.choice([8, 16])))
            for i in range(int(rng.integers(1, 4)))]
  lim = int(rng.choice([1, 2, 3, 5, 8, 16, 64, 1 << 12]))
  limits = (lim, int(rng.choice([lim, max(1, lim // 2)])))
  specs = _specs(tables, batch, limits, c["S"], c["combiner"], c["G"])
  feats = [_ragged(rng, batch, int(rng.integers(1, 10)), v)
           for _, v, _ in tables]
  weights = None
  if c["weighted"]:
    weights = []
    for f in feats:
      w = np.empty(len(f), dtype=object)
      for i, r in enumerate(f):
        w[i] = rng.uniform(0.1, 1, size=len(r)).astype(np.float32)
      weights.append(w)
  return c, specs, feats, weights, rng


def _check_csr(got, ref, c):
  rps, eids, sids, gns, nmb, stats = got
  assert nmb == ref.num_minibatches
  L, S, ns = c["L"], c["S"], c["S"] * c["G"]
  rpb = max(ns, 8)
  for name in ref.row_pointers:
    rp = rps[name].cpu().numpy()
    cs = eids[name].numel() // L
    if c["mb"]:
      for d in range(L):
        blk = slice(d * S * 64 * rpb, d * S * 64 * rpb + S * nmb * rpb)
        np.testing.assert_array_equal(rp[blk], ref.row_pointers[name][blk])
        end = min(-(-int(rp[blk].max()) // 8) * 8, cs)
        spans = [(d * cs, d * cs + end)]
    else:
      np.testing.assert_array_equal(rp, ref.row_pointers[name])
      per = cs // S
      spans = []
      for g, rs in enumerate(np.split(rp, L * S)):
        spans.append((g * per, g * per + int(rs[-1])))
    for got_d, exp_d in ((eids, ref.embedding_ids), (sids, ref.sample_ids),
                         (gns, ref.gains)):
      gv = got_d[name].cpu().numpy()
      ev = exp_d[name]
      for a, b in spans:
        np.testing.assert_array_equal(gv[a:b].view(np.int32),
                                      ev[a:b].view(np.int32))
    np.testing.assert_array_equal(stats.max_ids_per_partition[name],
                                  ref.max_ids_per_partition[name])
    np.testing.assert_array_equal(stats.max_unique_ids_per_partition[name],
                                  ref.max_unique_ids_per_partition[name])
    np.testing.assert_array_equal(stats.required_buffer_sizes[name],
                                  ref.required_buffer_sizes[name])
    assert stats.dropped_id_count[name] == ref.dropped_id_count[name]


def _check_lookup(got, ref, specs, c, rng):
  rps, eids, sids, gns, nmb, stats = got
  S = c["S"]
  for name in ref.row_pointers:
    st = next(fs.table_spec.stacked_table_spec for fs in specs
              if fs.table_spec.stacked_table_spec.stack_name == name)
    rows, dim = st.stack_vocab_size, st.stack_embedding_dim
    batch = st.total_sample_count
    table = rng.normal(size=(rows, dim)).astype(np.float32)
    kw = dict(max_ids_per_partition=st.max_ids_per_partition,
              max_unique_ids_per_partition=st.max_unique_ids_per_partition,
              num_sc_per_device=S, global_device_count=1,
              enable_minibatching=c["mb"],
              csr_num_entries=stats.num_entries[name])
    args = (rps[name], eids[name], sids[name], gns[name], np.int32(nmb))
    rargs = (ref.row_pointers[name], ref.embedding_ids[name],
             ref.sample_ids[name], ref.gains[name])
    lay = dict(num_sc_per_device=S, num_scs=S,
               num_minibatches=nmb if c["mb"] else 0)
    act = fwd_prim.tpu_sparse_dense_matmul_csr_primitive.bind(
        *args, torch.tensor(table).cuda(), device_batch_size=batch, **kw)
    np.testing.assert_allclose(
        act.cpu().numpy(), refcpu.sparse_dense_matmul(*rargs, table, batch,
                                                      **lay),
        rtol=RTOL, atol=ATOL)
    grad = rng.normal(size=(batch, dim)).astype(np.float32)
    tab = torch.tensor(table).cuda()
    acc = torch.full((rows, dim), 0.1, device="cuda")
    ada_prim.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
        *args, tab, acc, torch.tensor(grad).cuda(), 0.05, computation_name="a",
        csr_sorted_by_row=True, **kw)
    et, ea = refcpu.sparse_dense_matmul_grad(
        *rargs, grad, table, np.full((rows, dim), 0.1, np.float32),
        learning_rate=0.05, **lay)
    np.testing.assert_allclose(tab.cpu().numpy(), et, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(acc.cpu().numpy(), ea, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("chunk", range(6))
def test_random_cases(chunk):
  for seed in range(1000 + chunk * CASES_PER_TEST,
                    1000 + (chunk + 1) * CASES_PER_TEST):
    c, specs, feats, weights, rng = _draw(seed)
    kw = dict(num_sc_per_device=c["S"], allow_id_dropping=c["allow"],
              enable_minibatching=c["mb"])
    try:
      ref = refcpu.preprocess(feats, weights, specs, c["L"], c["G"], **kw)
    except RuntimeError:
      with pytest.raises(RuntimeError):
        pip.preprocess_sparse_dense_matmul_input(feats, weights, specs,
                                                 c["L"], c["G"], **kw)
      continue
    got = pip.preprocess_sparse_dense_matmul_input(feats, weights, specs,
                                                   c["L"], c["G"], **kw)
    try:
      _check_csr(got, ref, c)
      if c["L"] == 1 and c["G"] == 1:
        _check_lookup(got, ref, specs, c, rng)
    except AssertionError as e:
      raise AssertionError(f"seed {seed} case {c}") from e
