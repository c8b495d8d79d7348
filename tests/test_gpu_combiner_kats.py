"""The reference's combiner tests of the preprocessing, on the GPU.

Transcribed from lib/core/tests/pybind_input_preprocessing_test.py:
  test_combiner (:1695-1817): mean / sqrtn gains of weighted input equal
      the gains of the same input under the sum combiner with the weights
      normalised beforehand in numpy (w / sum(w), w / sqrt(sum(w^2))), on
      ragged and dense input, same seed (default_rng(12345)) and shapes;
  test_unity_weights_same_as_none (:1818-1869): explicit weights of 1.0 give
      the CSR of weights=None, for sum, mean and sqrtn.

Exactness. The reference's divisor is a sequential float loop over the row
(process_coo_tensors_impl.h:60-74). numpy's float32 sum is sequential for
fewer than 8 values and pairwise for 8 or more, so on the ragged rows (0-7
ids) the two agree and the gains must match bit for bit; on the dense rows
(8 ids each) numpy associates the sum differently, and rows 0 and 1 of this
seed sum to a value one ulp away from the sequential one (0.6413045 against
0.64130443 for row 0). There the gains are held to 2 ulp (a merged duplicate
sums two quotients), and separately to the CPU oracle bit for bit, which sums
sequentially as the reference does.
"""

import dataclasses

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
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position
from oracle import refcpu  # pylint: disable=g-import-not-at-top,wrong-import-position

NUM_SC = 4


def _spec(combiner, input_shape, output_shape, vocab, max_ids, name):
  table = embedding_spec.TableSpec(
      vocabulary_size=vocab, embedding_dim=8, initializer=None,
      optimizer=embedding_spec.SGDOptimizerSpec(learning_rate=0.001),
      combiner=combiner, name=name, max_ids_per_partition=max_ids,
      max_unique_ids_per_partition=max_ids)
  spec = embedding_spec.FeatureSpec(table_spec=table, input_shape=input_shape,
                                    output_shape=output_shape, name="feature")
  embedding.prepare_feature_specs_for_training(spec, global_device_count=1,
                                               num_sc_per_device=NUM_SC)
  return spec


def _compute_gains(weights, combiner):
  """Pre-normalised weights, as the reference test computes them (:1677)."""
  gains = []
  for w in weights:
    if combiner == "mean":
      w = w / np.sum(w)
    elif combiner == "sqrtn":
      w = w / np.sqrt(np.sum(np.square(w)))
    gains.append(w)
  if weights.ndim == 1:
    return np.array(gains, dtype=np.ndarray)
  return np.array(gains, dtype=np.float32)


def _run(features, weights, spec):
  rp, eid, sid, gains, *_ = pip.preprocess_sparse_dense_matmul_input(
      [features], None if weights is None else [weights], [spec],
      local_device_count=1, global_device_count=1, num_sc_per_device=NUM_SC,
      sharding_strategy=pip.ShardingStrategy.MOD, has_leading_dimension=False,
      allow_id_dropping=False, batch_number=42)
  name = spec.table_spec.name
  return tuple(x[name].cpu().numpy() for x in (rp, eid, sid, gains))


def _regions(rp, buf):
  """The compared region [0, rp_last) of every SparseCore's segment
  (lib/core/tests/test_utils.py:39-43)."""
  per_sc = buf.shape[0] // NUM_SC
  rp_per_sc = rp.shape[0] // NUM_SC
  return [buf[s * per_sc:s * per_sc + rp[(s + 1) * rp_per_sc - 1]]
          for s in range(NUM_SC)]


def _oracle(features, weights, spec):
  r = refcpu.preprocess([features], None if weights is None else [weights],
                        [spec], 1, 1, num_sc_per_device=NUM_SC)
  name = spec.table_spec.name
  return (r.row_pointers[name], r.embedding_ids[name], r.sample_ids[name],
          r.gains[name])


@pytest.mark.parametrize("combiner", ["mean", "sqrtn"])
@pytest.mark.parametrize("ragged", [True, False])
def test_combiner(combiner, ragged):
  spec = _spec(combiner, [4, None], [4, 8], 32, 32, "table")
  batch, max_ids_per_row, vocab = 4, 32 // 4, 32
  rng = np.random.default_rng(12345)
  feats, weights = [], []
  for _ in range(batch):
    n = max_ids_per_row
    if ragged:
      n = rng.integers(low=0, high=max_ids_per_row, size=1)
    feats.append(rng.integers(low=0, high=vocab, size=n).astype(np.int32))
    weights.append(rng.uniform(low=-1.0, high=1.0, size=n).astype(np.float32))
  if ragged:
    feats = np.array(feats, dtype=np.ndarray)
    weights = np.array(weights, dtype=np.ndarray)
  else:
    feats = np.array(feats, dtype=np.int32)
    weights = np.array(weights, dtype=np.float32)
  got = _run(feats, weights, spec)

  spec_sum = dataclasses.replace(
      spec, table_spec=dataclasses.replace(spec.table_spec, combiner="sum"))
  embedding.prepare_feature_specs_for_training(spec_sum, global_device_count=1,
                                               num_sc_per_device=NUM_SC)
  expected = _run(feats, _compute_gains(weights, combiner), spec_sum)

  np.testing.assert_array_equal(got[0], expected[0])
  for k in (1, 2):
    for a, b in zip(_regions(got[0], got[k]), _regions(got[0], expected[k])):
      np.testing.assert_array_equal(a, b)
  for a, b in zip(_regions(got[0], got[3]), _regions(got[0], expected[3])):
    if ragged:
      np.testing.assert_array_equal(a, b)
    else:
      # A divisor one ulp apart moves each quotient by at most one ulp; a
      # merged duplicate adds two of them (row 2 of this seed repeats id 15).
      np.testing.assert_array_max_ulp(a, b, maxulp=2)
  # Both runs equal the oracle on every written position, bit for bit.
  for run, w, sp in ((got, weights, spec),
                     (expected, _compute_gains(weights, combiner), spec_sum)):
    ref = _oracle(feats, w, sp)
    np.testing.assert_array_equal(run[0], ref[0])
    for k in (1, 2, 3):
      for a, b in zip(_regions(run[0], run[k]), _regions(run[0], ref[k])):
        np.testing.assert_array_equal(a.view(np.int32), b.view(np.int32))


SINGLETON = np.array([[5], [18], [0], [20], [6], [15], [12], [7], [3], [11],
                      [8], [26], [0], [18], [7], [2]], dtype=np.int32)
INPUT_FEATURES = np.array([[5, 18, 0, 20, 0, 2, 31, 3],
                           [18, 0, 20, 6, 1, 28, 5, 8],
                           [0, 20, 6, 15, 12, 7, 3, 11],
                           [18, 0, 7, 3, 6, 4, 19, 2]], dtype=np.int32)


@pytest.mark.parametrize("combiner", ["mean", "sqrtn", "sum"])
def test_unity_weights_same_as_none(combiner):
  spec = _spec(combiner, [4, 4], [4, 8], 32, 16, "table")
  with_w = _run(INPUT_FEATURES, np.ones_like(INPUT_FEATURES, np.float32),
                spec)
  without = _run(INPUT_FEATURES, None, spec)
  np.testing.assert_array_equal(with_w[0], without[0])
  for k in (1, 2, 3):
    for a, b in zip(_regions(with_w[0], with_w[k]),
                    _regions(with_w[0], without[k])):
      np.testing.assert_array_equal(a.view(np.int32), b.view(np.int32))
