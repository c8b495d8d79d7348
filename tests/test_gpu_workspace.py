"""The measured preprocessing workspace is enough, to the byte.

scemb_preprocess_workspace_size runs the call's code in measuring mode; a
call given exactly that many bytes must succeed (one call for all stacks
carves each stack exactly its measured slice). The cases take every route
with inputs large enough that each scan spans several tiles, and compare the
outputs with those of a call given a roomy workspace.
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


def _stack(rng, weighted, limit):
  batch, vocab = 4096, 50_000
  t = embedding_spec.TableSpec(
      name="t", vocabulary_size=vocab, embedding_dim=8,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.1),
      combiner="mean" if weighted else "sum", max_ids_per_partition=limit,
      max_unique_ids_per_partition=limit)
  specs = [embedding_spec.FeatureSpec(
      name="f", table_spec=t, input_shape=[batch, 1],
      output_shape=[batch, 8])]
  embedding.prepare_feature_specs_for_training(specs, 1, 1)
  lens = rng.integers(0, 30, size=batch)
  ids = np.empty(batch, dtype=object)
  ws = np.empty(batch, dtype=object)
  for i, n in enumerate(lens):
    ids[i] = (rng.zipf(1.2, size=int(n)) % vocab).astype(np.int32)
    ws[i] = rng.uniform(0.1, 2, size=int(n)).astype(np.float32)
  (name, metas), = pip.get_stacked_table_metadata(specs).items()
  feat = pip._to_device_feature(ids, ws if weighted else None)  # pylint: disable=protected-access
  return metas, feat


def _call(metas, feat, weighted, extra, rp_words, **kw):
  """One call with `extra` bytes beyond the measured workspace: its first
  `rp_words` row pointers, the CSR entries below the largest of them, the
  initialised stats words and the view (0 rp_words: stats only)."""
  call, res = pip._prepare_stack(  # pylint: disable=protected-access
      [feat], metas, local_device_count=1, global_device_count=1,
      num_sc_per_device=1, allow_id_dropping=False, has_weights=weighted,
      **kw)
  buf = torch.empty(call.need + extra + 256, dtype=torch.uint8, device="cuda")
  base = (_native.ptr(buf) + 255) // 256 * 256
  rc = _native.load_library().scemb_preprocess_stacked_table(
      call.structs, call.num_features, ctypes.byref(call.opts),
      ctypes.byref(call.out), base, call.need + extra,
      _native.stream_handle())
  torch.cuda.synchronize()
  assert rc == 0, _native.load_library().scemb_last_error().decode()
  rp, eid, sid, gains, stats, (_, _, _, off), view = res
  out = [stats[:off + 2 * pip._NUM_COUNTERS].cpu().numpy()]  # pylint: disable=protected-access
  if rp_words:
    rp = rp.reshape(-1)[:rp_words]
    n = int(rp.max().item())  # minibatches end at their own row pointers
    out += [rp.cpu().numpy(), eid[:n].cpu().numpy(), sid[:n].cpu().numpy(),
            gains[:n].cpu().numpy().view(np.int32)]
  if view is not None:
    out += [view[0].cpu().numpy(), view[1].cpu().numpy()]
  return out


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("route", ["extraction", "after_sort", "mb0", "mb1",
                                   "mb2"])
def test_exact_workspace_suffices(route, weighted):
  rng = np.random.default_rng(3 + weighted)
  limit = 1 << 17
  metas, feat = _stack(rng, weighted, limit)
  kw = {}
  old = pip.PREPROCESS_FLAGS
  if route == "after_sort":
    pip.PREPROCESS_FLAGS = _native.PREPROCESS_GROUP_AFTER_SORT
  if route.startswith("mb"):
    kw = dict(enable_minibatching=True, minibatching_pass=int(route[2]),
              minibatching_split=0b101 if route == "mb2" else 0)
  kw["build_view"] = route != "mb1"
  # Eight row pointers per minibatch (one partition, padded to eight); the
  # bucket pass writes none, pass 2 writes its three minibatches.
  rp_words = {"mb1": 0, "mb2": 3 * 8}.get(route, 8)
  try:
    exact = _call(metas, feat, weighted, 0, rp_words, **kw)
    roomy = _call(metas, feat, weighted, 1 << 20, rp_words, **kw)
  finally:
    pip.PREPROCESS_FLAGS = old
  for a, b in zip(exact, roomy):
    np.testing.assert_array_equal(a, b)
  if rp_words:
    assert exact[2].size > 2048  # several scan tiles
