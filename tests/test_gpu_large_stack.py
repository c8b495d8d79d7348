"""A stack too long for the grouped scan: both grouping routes agree.

The route that merges duplicates at extraction scans each radix pass's
digit-count matrix with one grouped scan of at most 8,192 tiles of 2,048
counts. A stack whose matrix is longer (here 2.2M samples of 64 ids, 140.8M
ids under 30-bit keys: 68,750 tiles x 256 digits, 17.6M counts) scans it
with the recursive ExclusiveScan instead. Every seventh row holds a hot id
twice, which the extraction merges. This case runs such a stack through both routes and
compares the row pointers, the CSR entries and the stats on the device, bit
for bit (the after-sort route is the one the oracle pins at small sizes).
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


def _run(flags, ids, specs):
  old = pip.PREPROCESS_FLAGS
  pip.PREPROCESS_FLAGS = flags
  try:
    rps, eids, sids, gns, pending = pip.enqueue_preprocessing(
        [ids], None, specs, 1, 1, num_sc_per_device=1)
    torch.cuda.synchronize()
  finally:
    pip.PREPROCESS_FLAGS = old
  (name,) = rps
  n = int(rps[name][0].item())
  return (rps[name].clone(), eids[name][:n].clone(), sids[name][:n].clone(),
          gns[name][:n].view(torch.int32).clone(),
          pending.stats_buffer.clone())


def test_stack_longer_than_the_grouped_scan():
  batch, valency = 2_200_000, 64
  total = batch * valency
  vocab = 1 << 30
  t = embedding_spec.TableSpec(
      name="big", vocabulary_size=vocab, embedding_dim=8,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner="sum",
      max_ids_per_partition=total + 8, max_unique_ids_per_partition=total + 8)
  specs = [embedding_spec.FeatureSpec(
      name="f", table_spec=t, input_shape=[batch, valency],
      output_shape=[batch, 8])]
  embedding.prepare_feature_specs_for_training(specs, 1, 1)
  gen = torch.Generator(device="cuda")
  gen.manual_seed(5)
  ids = torch.randint(0, vocab, (batch, valency), dtype=torch.int32,
                      device="cuda", generator=gen)
  # A hot id twice in every seventh row: merged copies, and equal keys that
  # span many tiles.
  ids[::7, 0] = 12345
  ids[::7, 1] = 12345
  a = _run(0, ids, specs)
  b = _run(_native.PREPROCESS_GROUP_AFTER_SORT, ids, specs)
  # One entry per distinct id of a row (random ids also repeat now and then).
  srt = torch.sort(ids, dim=1).values
  distinct = int((srt[:, 1:] != srt[:, :-1]).sum().item()) + batch
  del srt
  assert distinct < total - batch // 7
  assert int(a[0][0].item()) == distinct
  for x, y, what in zip(a, b, ("row pointers", "ids", "samples", "gains",
                                "stats")):
    assert x.shape == y.shape, what
    words = x.shape[0] - 2 if what == "stats" else x.shape[0]
    assert torch.equal(x[:words], y[:words]), what
  # Sorted by column, as the CSR requires.
  e = a[1].to(torch.int64)
  assert bool((e[1:] >= e[:-1]).all())
  del a, b, ids
  torch.cuda.empty_cache()
