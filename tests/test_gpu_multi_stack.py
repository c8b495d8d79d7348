"""Several stacked tables in one library call equal one call per stack.

enqueue_preprocessing hands every stack of a batch to
scemb_preprocess_stacked_tables, which runs each stage of the stacks that
merge duplicates at extraction as one grouped launch (up to eight stacks per
launch) and the other stacks one after another. These cases run the same
inputs once through that call and once with every stack sent to
scemb_preprocess_stacked_table on its own, and compare the row pointers, the
written CSR entries, the whole stats block and the sample views bit for bit.
They cover more stacks than one grouped launch holds, a stack whose rows are
too long for the extraction route next to ones that take it, a stack with no
ids, weighted stacks, and several SparseCores. Correctness of the single-stack
call itself is the parity tests' job (oracle).
"""

import ctypes

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


def _specs(vocabs, batch, combiner, num_sc, limit=4096):
  specs = []
  for i, vocab in enumerate(vocabs):
    t = embedding_spec.TableSpec(
        name=f"t{i}", vocabulary_size=vocab, embedding_dim=8,
        initializer=embedding_spec.zeros,
        optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner=combiner,
        max_ids_per_partition=limit, max_unique_ids_per_partition=limit)
    specs.append(embedding_spec.FeatureSpec(
        name=f"f{i}", table_spec=t, input_shape=[batch, 1],
        output_shape=[batch, 8]))
  embedding.prepare_feature_specs_for_training(specs, 1, num_sc)
  return specs


def _ragged(rng, lens, vocab):
  out = np.empty(len(lens), dtype=object)
  for i, n in enumerate(lens):
    # Skewed ids, so that rows repeat ids and the merging has work.
    out[i] = (rng.zipf(1.3, size=int(n)) % vocab).astype(np.int32)
  return out


def _weights(rng, feats):
  ws = []
  for f in feats:
    w = np.empty(len(f), dtype=object)
    for i, r in enumerate(f):
      w[i] = rng.uniform(0.05, 2, size=len(r)).astype(np.float32)
    ws.append(w)
  return ws


def _one_by_one(calls):
  """_preprocess_stacks with each stack sent to the single-stack call."""
  lib = _native.load_library()
  for c in calls:
    ws = _native.WORKSPACE.get(c.need)
    _native.check(lib.scemb_preprocess_stacked_table(
        c.structs, c.num_features, ctypes.byref(c.opts), ctypes.byref(c.out),
        _native.ptr(ws), ws.numel(), _native.stream_handle()))


def _run(feats, weights, specs, num_sc, view, one_by_one):
  grouped = pip._preprocess_stacks  # pylint: disable=protected-access
  if one_by_one:
    pip._preprocess_stacks = _one_by_one  # pylint: disable=protected-access
  try:
    views = {} if view else None
    rps, eids, sids, gns, pending = pip.enqueue_preprocessing(
        feats, weights, specs, 1, 1, num_sc_per_device=num_sc,
        sample_views=views)
    torch.cuda.synchronize()
  finally:
    pip._preprocess_stacks = grouped  # pylint: disable=protected-access
  out = {}
  for name in rps:
    rp = rps[name].cpu().numpy().reshape(-1)
    per = eids[name].numel() // num_sc
    spans = [(g * per, g * per + int(rs[-1]))
             for g, rs in enumerate(np.split(rp, num_sc))]
    written = [np.concatenate([x.cpu().numpy().reshape(-1).view(np.int32)[a:b]
                               for a, b in spans])
               for x in (eids[name], sids[name], gns[name])]
    out[name] = dict(rp=rp, eid=written[0], sid=written[1], gain=written[2])
    if view:
      k, e = views[name]
      out[name]["vkeys"] = k.cpu().numpy()
      out[name]["ventries"] = e.cpu().numpy()
  out["stats"] = pending.stats_buffer.cpu().numpy()
  return out


def _compare(a, b):
  """Every stack's arrays, then the stats block stack by stack (its words
  named by stack and offset in the message)."""
  assert a.keys() == b.keys()
  for name in a:
    if name == "stats":
      continue
    for key in a[name]:
      np.testing.assert_array_equal(a[name][key], b[name][key],
                                    err_msg=f"{name} {key}")
  stacks = len(a) - 1
  words = a["stats"].size // stacks
  # Each stack's slice ends with two words of alignment padding that the
  # library does not write (_stats_words); the rest it initialises.
  for s in range(stacks):
    x = a["stats"][s * words:(s + 1) * words - 2]
    y = b["stats"][s * words:(s + 1) * words - 2]
    bad = np.nonzero(x != y)[0]
    assert bad.size == 0, (
        f"stats of stack {s}: words {bad.tolist()} are "
        f"{x[bad].tolist()}, expected {y[bad].tolist()}")


@pytest.mark.parametrize("weighted", [False, True])
def test_ten_stacks_in_one_call_match_one_call_each(weighted):
  """Ten stacks (two grouped launches per stage), one of them with rows too
  long for the extraction route and one with no ids at all."""
  rng = np.random.default_rng(7 + weighted)
  batch = 512
  vocabs = [10_000 + 3_000 * i for i in range(10)]
  specs = _specs(vocabs, batch, "sqrtn" if weighted else "mean", 1,
                 limit=batch * 1100)
  feats = []
  for i, vocab in enumerate(vocabs):
    if i == 3:
      lens = np.full(batch, 0)
      lens[5] = 1000  # longer than the extraction route's staging
      lens[100] = 3
    elif i == 6:
      lens = np.zeros(batch, np.int64)  # no ids
    else:
      lens = rng.integers(0, 40, size=batch)
    feats.append(_ragged(rng, lens, vocab))
  weights = _weights(rng, feats) if weighted else None
  one = _run(feats, weights, specs, 1, True, one_by_one=True)
  many = _run(feats, weights, specs, 1, True, one_by_one=False)
  _compare(many, one)
  assert int(one["t3"]["rp"][-1]) > 0 and int(one["t6"]["rp"][-1]) == 0


def test_several_sparsecores_without_views():
  """Four SparseCores: stacks of different key widths in one call."""
  rng = np.random.default_rng(11)
  batch = 1024
  vocabs = [64, 5_000, 300_000, 2_000_000]
  specs = _specs(vocabs, batch, "sum", 4, limit=batch * 64)
  feats = [_ragged(rng, rng.integers(1, 30, size=batch), v) for v in vocabs]
  one = _run(feats, None, specs, 4, False, one_by_one=True)
  many = _run(feats, None, specs, 4, False, one_by_one=False)
  _compare(many, one)
