"""The two grouping routes of the GPU preprocessing give identical outputs.

Where the features' sample rows are disjoint and neither id dropping nor
minibatching is on, the library merges duplicate ids of an input row while
extracting and sorts the distinct entries; otherwise it sorts every id and
merges duplicates after the sort (SCEMB_PREPROCESS_GROUP_AFTER_SORT forces
this route). Every case here runs through both and compares the row
pointers, the written CSR entries, the whole stats block (counters included)
and, on one device, the sample view, bit for bit. The after-sort route is
itself checked against the oracle by the parity tests; the cases below
stress what the extraction route does differently: rows longer than its LDS
staging, rows crossing blocks, heavy duplication, weighted divisors, dense
inputs of several ids per row, ids outside the table, empty rows and
features, several SparseCores and devices, and 64-bit keys.
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


from jax_tpu_embedding.sparsecore import _native  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position


def _specs(tables, batch, combiner, num_sc, devices, limit):
  specs = []
  for name, vocab in tables:
    t = embedding_spec.TableSpec(
        name=name, vocabulary_size=vocab, embedding_dim=8,
        initializer=embedding_spec.zeros,
        optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner=combiner,
        max_ids_per_partition=limit, max_unique_ids_per_partition=limit)
    specs.append(embedding_spec.FeatureSpec(
        name=f"f_{name}", table_spec=t, input_shape=[batch, 1],
        output_shape=[batch, 8]))
  embedding.prepare_feature_specs_for_training(specs, devices, num_sc)
  return specs


def _ragged(rng, lens, vocab, bad=0.0):
  out = np.empty(len(lens), dtype=object)
  for i, n in enumerate(lens):
    ids = rng.integers(0, vocab, size=int(n)).astype(np.int32)
    if bad:
      ids[rng.random(int(n)) < bad] = -3
    out[i] = ids
  return out


def _weights(rng, feats):
  ws = []
  for f in feats:
    if isinstance(f, np.ndarray) and f.dtype != object:
      ws.append(rng.uniform(0.05, 2, size=f.shape).astype(np.float32))
      continue
    w = np.empty(len(f), dtype=object)
    for i, r in enumerate(f):
      w[i] = rng.uniform(0.05, 2, size=len(r)).astype(np.float32)
    ws.append(w)
  return ws


def _run(flags, feats, weights, specs, L, G, S, view):
  old = pip.PREPROCESS_FLAGS
  pip.PREPROCESS_FLAGS = flags
  try:
    views = {} if view else None
    rps, eids, sids, gns, pending = pip.enqueue_preprocessing(
        feats, weights, specs, L, G, num_sc_per_device=S, sample_views=views)
    torch.cuda.synchronize()
  finally:
    pip.PREPROCESS_FLAGS = old
  out = {}
  for name in rps:
    rp = rps[name].cpu().numpy().reshape(-1)
    cs = eids[name].numel() // L
    per = cs // S
    spans = [(g * per, g * per + int(rs[-1]))
             for g, rs in enumerate(np.split(rp, L * S))]
    written = [np.concatenate([x.cpu().numpy().reshape(-1).view(np.int32)[a:b]
                               for a, b in spans])
               for x in (eids[name], sids[name], gns[name])]
    out[name] = dict(rp=rp, eid=written[0], sid=written[1], gain=written[2])
    if view:
      k, e = views[name]
      out[name]["vkeys"] = k.cpu().numpy()
      out[name]["ventries"] = e.cpu().numpy()
  for name, stats_dev, *_, off, _ in pending:
    # The words the library initialises: stats, then six int64 counters.
    words = stats_dev.cpu().numpy()[:off + 12]
    out[name]["stats"] = words
    out[name]["counters"] = words[off:].copy().view(np.int64)
  return out


def _compare(case, feats, weights, specs, L=1, G=1, S=1, view=None):
  if view is None:
    view = L == 1 and G == 1
  a = _run(0, feats, weights, specs, L, G, S, view)
  b = _run(_native.PREPROCESS_GROUP_AFTER_SORT, feats, weights, specs, L, G,
           S, view)
  assert a.keys() == b.keys()
  for name in a:
    for k in a[name]:
      np.testing.assert_array_equal(a[name][k], b[name][k],
                                    err_msg=f"{case} {name} {k}")
  return a


@pytest.mark.parametrize("combiner", ["sum", "mean", "sqrtn"])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("num_sc", [1, 4])
def test_ragged_heavy_duplicates(combiner, weighted, num_sc):
  rng = np.random.default_rng(7 + num_sc)
  batch = 512
  tables = [("a", 40), ("b", 3000), ("c", 7)]
  specs = _specs(tables, batch, combiner, num_sc, 1, 1 << 14)
  feats = [_ragged(rng, rng.integers(0, 60, size=batch), v)
           for _, v in tables]
  weights = _weights(rng, feats) if weighted else None
  out = _compare((combiner, weighted, num_sc), feats, weights, specs,
                 S=num_sc)
  # Duplicates were merged: fewer grouped entries than ids.
  ids = sum(len(r) for f in feats for r in f)
  assert 0 < sum(int(v["counters"][3]) for v in out.values()) < ids


@pytest.mark.parametrize("weighted", [False, True])
def test_rows_up_to_the_route_limit(weighted):
  """Rows of up to 896 ids (the longest the extraction route takes): a
  block's rows then just fit its LDS staging; row boundaries fall inside and
  across blocks."""
  rng = np.random.default_rng(12)
  batch = 96
  lens = rng.integers(0, 40, size=batch)
  lens[[3, 4, 17, 40, 41, 90]] = [896, 896, 700, 895, 1, 896]
  specs = _specs([("a", 900)], batch, "sqrtn", 1, 1, 1 << 16)
  feats = [_ragged(rng, lens, 900)]
  weights = _weights(rng, feats) if weighted else None
  _compare(("limit", weighted), feats, weights, specs)


@pytest.mark.parametrize("weighted", [False, True])
def test_rows_longer_than_the_staging(weighted, monkeypatch):
  """Rows of up to 5,000 ids normally go the after-sort route. With a row
  length hint that understates them, the extraction route runs with blocks
  whose rows do not fit LDS and reads them from memory: still the same
  outputs (the hint only picks the route)."""
  rng = np.random.default_rng(11)
  batch = 64
  lens = rng.integers(0, 40, size=batch)
  lens[[3, 17, 40]] = [5000, 2100, 2047]
  specs = _specs([("a", 900)], batch, "mean", 1, 1, 1 << 16)
  feats = [_ragged(rng, lens, 900)]
  weights = _weights(rng, feats) if weighted else None
  _compare(("long", weighted), feats, weights, specs)
  resolve = pip._resolve_feature  # pylint: disable=protected-access

  def understated(f):
    f = resolve(f)
    f.max_row_length = 2
    return f

  monkeypatch.setattr(pip, "_resolve_feature", understated)
  _compare(("long, hint 2", weighted), feats, weights, specs)


@pytest.mark.parametrize("valency", [1, 3, 50, 3000])
def test_dense_rows(valency):
  rng = np.random.default_rng(valency)
  batch = 256 if valency < 1000 else 16
  specs = _specs([("a", 500), ("b", 20)], batch, "sqrtn", 2, 1, 1 << 16)
  feats = [rng.integers(0, v, size=(batch, valency)).astype(np.int32)
           for v in (500, 20)]
  _compare(("dense", valency), feats, _weights(rng, feats), specs, S=2)


def test_invalid_ids_counted_alike():
  rng = np.random.default_rng(3)
  batch = 256
  specs = _specs([("a", 100), ("b", 60)], batch, "sum", 1, 1, 1 << 14)
  feats = [_ragged(rng, rng.integers(0, 12, size=batch), 100, bad=0.1),
           _ragged(rng, rng.integers(0, 12, size=batch), 60)]
  out = _compare("invalid", feats, None, specs)
  bad = sum(int(np.sum(r < 0)) for r in feats[0])
  assert bad > 0
  assert sum(int(v["counters"][2]) for v in out.values()) == bad


def test_empty_rows_and_features():
  rng = np.random.default_rng(5)
  batch = 128
  specs = _specs([("a", 50), ("b", 50), ("c", 50)], batch, "mean", 2, 1,
                 1 << 12)
  lens = np.zeros(batch, np.int64)
  lens[::9] = rng.integers(1, 6, size=lens[::9].size)
  feats = [_ragged(rng, lens, 50), _ragged(rng, np.zeros(batch, np.int64), 50),
           _ragged(rng, rng.integers(0, 4, size=batch), 50)]
  _compare("empty", feats, _weights(rng, feats), specs, S=2)


@pytest.mark.parametrize("L,G,S", [(1, 2, 2), (2, 2, 1), (2, 2, 4)])
def test_several_devices(L, G, S):
  rng = np.random.default_rng(L * 10 + G + S)
  batch = 256 * G
  tables = [("a", 700), ("b", 90)]
  specs = _specs(tables, batch, "mean", S, G, 1 << 14)
  feats = [_ragged(rng, rng.integers(0, 20, size=batch), v)
           for _, v in tables]
  _compare(("devices", L, G, S), feats, _weights(rng, feats), specs, L=L,
           G=G, S=S)


def test_wide_keys():
  """A vocabulary of 2^30 rows over two devices of four SparseCores makes
  the sort key wider than 31 bits."""
  rng = np.random.default_rng(9)
  batch = 256
  vocab = 1 << 30
  specs = _specs([("a", vocab)], batch, "sum", 4, 2, 1 << 14)
  lens = rng.integers(0, 10, size=batch)
  f = _ragged(rng, lens, 64)
  hot = rng.integers(0, vocab, size=64).astype(np.int32)
  for i in range(batch):
    f[i] = hot[f[i] % 64]
  _compare("wide", [f], None, specs, L=2, G=2, S=4)


def test_view_tail_and_many_stacks():
  """Several stacks of one call (grouped launches) with their sample views."""
  rng = np.random.default_rng(21)
  batch = 1024
  specs = []
  feats = []
  for k, (v, d) in enumerate([(300, 8), (5000, 16), (40, 32)]):
    t = embedding_spec.TableSpec(
        name=f"s{k}", vocabulary_size=v, embedding_dim=d,
        initializer=embedding_spec.zeros,
        optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner="sqrtn",
        max_ids_per_partition=1 << 15, max_unique_ids_per_partition=1 << 15)
    specs.append(embedding_spec.FeatureSpec(
        name=f"g{k}", table_spec=t, input_shape=[batch, 1],
        output_shape=[batch, d]))
    feats.append(_ragged(rng, rng.integers(0, 30, size=batch), v))
  embedding.prepare_feature_specs_for_training(specs, 1, 1)
  _compare("stacks", feats, _weights(rng, feats), specs)
