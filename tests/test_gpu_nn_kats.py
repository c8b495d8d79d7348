"""The reference's embedding-API tests with exact answers, on the GPU.

Transcribed from the reference (paths under jax_tpu_embedding/sparsecore/):
  lib/nn/tests/tpu_sparse_dense_matmul_test.py:587-689
      (test_sparse_dense_matmul_single_chip): two features on two tables
      whose rows hold their own ids; every activation row is the sum of the
      sample's ids.
  lib/nn/tests/tpu_sparse_dense_matmul_grad_test.py:236-667
      (test_sparse_dense_matmul_one_chip_unsharded): four tables (SGD, SGD,
      Adagrad, F2A) updated with unit gradients; the SGD tables must equal
      `row - 0.01 * count` exactly, Adagrad and F2A the reference's literal
      tables and slots (F2A to the reference's rtol / atol 1e-5).
Both go through the whole API: prepare_feature_specs_for_training,
preprocess_sparse_dense_matmul_input (GPU preprocessing), then
tpu_sparse_dense_matmul / tpu_sparse_dense_matmul_grad. Tables are given in
the stacked (MOD-sharded) layout, built here row by row: logical row r of a
table sits at row (r % S) * (V / S) + r // S for S SparseCores, so the
layout itself is checked too. The reference runs these with 4 SparseCores;
1 and 2 are added, with the literal expectations moved to that layout.

The reference's multi-chip variants of these tests need a second device and
the cross-device exchange, which this one-GPU build does not have.
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


from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position


def _ragged(rows):
  return np.array([np.array(r, dtype=np.int32) for r in rows], dtype=object)


INPUT_A = _ragged([[5, 4, 2], [3], [9], [1, 9, 16], [6, 12, 1, 10], [12, 19],
                   [0, 15, 2, 25, 25], [4, 28, 25], [15, 0], [13], [11],
                   [7, 1], [8, 9], [14, 14, 14], [2, 28], [10, 16]])
INPUT_B = _ragged([[50, 40, 20], [33], [59], [1, 9, 16], [6, 12, 1, 10],
                   [12, 19], [0, 15, 2, 25, 25], [4, 28, 25], [50, 51, 0],
                   [10, 50, 60], [11, 12, 13], [61, 60], [58, 2],
                   [41, 41, 50], [2, 58], [10, 16]])
INPUT_CD = np.array([[5], [3], [9], [1], [6], [12], [0], [4], [15], [13],
                     [11], [7], [8], [14], [2], [10]], dtype=np.int32)


def _shard(logical, num_sc):
  """MOD layout of a [V, D] table for one device, row by row."""
  v = logical.shape[0]
  out = np.empty_like(logical)
  for r in range(v):
    out[(r % num_sc) * (v // num_sc) + r // num_sc] = logical[r]
  return out


def _unshard(sharded, num_sc):
  v = sharded.shape[0]
  out = np.empty_like(sharded)
  for r in range(v):
    out[r] = sharded[(r % num_sc) * (v // num_sc) + r // num_sc]
  return out


def _row_table(vocab, dim):
  return np.tile(np.arange(vocab, dtype=np.float32)[:, None], (1, dim))


def _cuda(x):
  return torch.tensor(np.ascontiguousarray(x)).cuda()


# --- tpu_sparse_dense_matmul_test.py:587-689 -------------------------------

EXPECTED_ACT_A = np.array([11, 3, 9, 26, 29, 31, 67, 57, 15, 13, 11, 8, 17,
                           42, 30, 26], np.float32)


@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("unstack_primitive", [False, True])
def test_sparse_dense_matmul_single_chip(num_sc, unstack_primitive):
  opt = embedding_spec.SGDOptimizerSpec()
  # The reference's limit of 16 ids per partition fits its 4 SparseCores;
  # with fewer, each partition holds more of the 34 ids.
  limit = 16 if num_sc == 4 else 64
  ta = embedding_spec.TableSpec(
      vocabulary_size=32, embedding_dim=6, initializer=None, optimizer=opt,
      combiner="sum", name="table_a", max_ids_per_partition=limit,
      max_unique_ids_per_partition=limit)
  tb = embedding_spec.TableSpec(
      vocabulary_size=64, embedding_dim=16, initializer=None, optimizer=opt,
      combiner="sum", name="table_b", max_ids_per_partition=limit,
      max_unique_ids_per_partition=limit)
  feature_specs = {
      "feature_spec_a": embedding_spec.FeatureSpec(
          table_spec=ta, input_shape=(16, 1), output_shape=(16, 6),
          name="feature_spec_a"),
      "feature_spec_b": embedding_spec.FeatureSpec(
          table_spec=tb, input_shape=(16, 1), output_shape=(16, 16),
          name="feature_spec_b"),
  }
  embedding.prepare_feature_specs_for_training(
      feature_specs, global_device_count=1, num_sc_per_device=num_sc)
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      {"feature_spec_a": INPUT_A, "feature_spec_b": INPUT_B},
      features_weights=None, feature_specs=feature_specs,
      local_device_count=1, global_device_count=1, num_sc_per_device=num_sc,
      sharding_strategy="MOD", batch_number=42)
  variables = {
      "table_a": embedding.EmbeddingVariables(
          table=_cuda(_shard(_row_table(32, 8), num_sc)), slot=()),
      "table_b": embedding.EmbeddingVariables(
          table=_cuda(_shard(_row_table(64, 16), num_sc)), slot=()),
  }
  leaves = (feature_specs["feature_spec_a"], feature_specs["feature_spec_b"])
  acts = embedding.tpu_sparse_dense_matmul(
      pre, variables, leaves, global_device_count=1, sharding_strategy="MOD",
      num_sc_per_device=num_sc,
      use_activation_unstack_primitive=unstack_primitive)
  assert len(acts) == 2
  np.testing.assert_array_equal(
      acts[0].cpu().numpy(), np.tile(EXPECTED_ACT_A[:, None], (1, 6)))
  expected_b = np.array([sum(r) for r in INPUT_B], np.float32)
  np.testing.assert_array_equal(acts[1].cpu().numpy(),
                                np.tile(expected_b[:, None], (1, 16)))


# --- tpu_sparse_dense_matmul_grad_test.py:236-667 --------------------------

# Table c after one Adagrad step, in the 4-SparseCore layout of the
# reference (rows 0, 4, 8, ... first), and its accumulator.
EXPECTED_TABLE_C_SC4 = np.array(
    [-1.000e-02, 3.990e00, 7.990e00, 1.199e01, 1.600e01, 2.000e01, 2.400e01,
     2.800e01, 9.900e-01, 4.990e00, 8.990e00, 1.299e01, 1.700e01, 2.100e01,
     2.500e01, 2.900e01, 1.990e00, 5.990e00, 9.990e00, 1.399e01, 1.800e01,
     2.200e01, 2.600e01, 3.000e01, 2.990e00, 6.990e00, 1.099e01, 1.499e01,
     1.900e01, 2.300e01, 2.700e01, 3.100e01], np.float32)
EXPECTED_ACC_C_SC4 = np.array(
    [1.0] * 4 + [0.0] * 4 + [1.0] * 4 + [0.0] * 4 + [1.0] * 4 + [0.0] * 4 +
    [1.0] * 4 + [0.0] * 4, np.float32)
# Table d after one F2A step and its slots, in the logical row order.
EXPECTED_TABLE_D = np.array(
    [-9.534626e-03, 9.904354e-01, 1.990415e00, 2.990395e00, 3.990375e00,
     4.990355e00, 5.990335e00, 6.990315e00, 7.990295e00, 8.990275e00,
     9.990255e00, 1.099024e01, 1.199022e01, 1.299020e01, 1.399018e01,
     1.499016e01, 1.600000e01, 1.700000e01, 1.800000e01, 1.900000e01,
     2.000000e01, 2.100000e01, 2.200000e01, 2.300000e01, 2.400000e01,
     2.500000e01, 2.600000e01, 2.700000e01, 2.800000e01, 2.900000e01,
     3.000000e01, 3.100000e01], np.float32)
EXPECTED_ACC_D = np.array([1.1] * 16 + [0.1] * 16, np.float32)
EXPECTED_STEP_D = np.array([1.0] * 16 + [0.0] * 16, np.float32)


def _count(rows, v):
  return sum(int(x == v) for r in rows for x in r)


@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("stacking_primitive", [False, True])
def test_sparse_dense_matmul_grad_one_chip_unsharded(num_sc,
                                                     stacking_primitive):
  def table(name, vocab, dim, opt):
    return embedding_spec.TableSpec(vocabulary_size=vocab, embedding_dim=dim,
                                    initializer=None, optimizer=opt,
                                    combiner="sum", name=name)

  f2a = embedding_spec.F2AOptimizerSpec(
      learning_rate=0.01, rho=0.5, initial_accumulator_value=0.1,
      initial_local_step_value=0.0, l1_regularization_strength=0.001,
      l2_regularization_strength=0.002, max_lr_multiplier=100.0)
  tables = {
      "a": table("table_a", 32, 4, embedding_spec.SGDOptimizerSpec(0.01)),
      "b": table("table_b", 64, 6, embedding_spec.SGDOptimizerSpec(0.01)),
      "c": table("table_c", 32, 18,
                 embedding_spec.AdagradOptimizerSpec(learning_rate=0.01)),
      "d": table("table_d", 32, 8, f2a),
  }
  feature_specs = {
      f"feature_spec_{k}": embedding_spec.FeatureSpec(
          table_spec=t, input_shape=(16, 1),
          output_shape=(16, t.embedding_dim), name=f"feature_spec_{k}")
      for k, t in tables.items()}
  embedding.prepare_feature_specs_for_training(
      feature_specs, num_sc_per_device=num_sc, global_device_count=1)
  inputs = {"feature_spec_a": INPUT_A, "feature_spec_b": INPUT_B,
            "feature_spec_c": INPUT_CD, "feature_spec_d": INPUT_CD}
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      inputs, features_weights=None, feature_specs=feature_specs,
      local_device_count=1, global_device_count=1, num_sc_per_device=num_sc,
      sharding_strategy="MOD", batch_number=42)

  dims = {"a": 8, "b": 8, "c": 24, "d": 8}
  vocabs = {"a": 32, "b": 64, "c": 32, "d": 32}
  sharded = {k: _shard(_row_table(vocabs[k], dims[k]), num_sc)
             for k in tables}
  variables = {
      "table_a": (_cuda(sharded["a"]),),
      "table_b": (_cuda(sharded["b"]),),
      "table_c": (_cuda(sharded["c"]), _cuda(np.zeros_like(sharded["c"]))),
      "table_d": (_cuda(sharded["d"]),
                  _cuda(np.full_like(sharded["d"], 0.1)),
                  _cuda(np.zeros_like(sharded["d"]))),
  }
  grads = {f"feature_spec_{k}": torch.ones(16, t.embedding_dim).cuda()
           for k, t in tables.items()}
  kwargs = {"global_device_count": 1} if stacking_primitive else {}
  out = embedding.tpu_sparse_dense_matmul_grad(
      grads, pre, variables, feature_specs, sharding_strategy="MOD",
      num_sc_per_device=num_sc,
      use_gradient_stacking_primitive=stacking_primitive, **kwargs)

  for k, rows, dim in (("a", INPUT_A, 4), ("b", INPUT_B, 6)):
    expected = np.zeros((vocabs[k], dim), np.float32)
    for i, row in enumerate(sharded[k]):
      v = row[0]
      expected[i] = np.full((dim,), v - (_count(rows, v) * 0.01), np.float32)
    np.testing.assert_array_equal(
        out[f"table_{k}"][0].cpu().numpy()[:, :dim], expected)

  def moved(sc4_values, dim):
    logical = _unshard(np.tile(sc4_values[:, None], (1, dim)), 4)
    return _shard(logical, num_sc)

  np.testing.assert_array_equal(out["table_c"][0].cpu().numpy()[:, :18],
                                moved(EXPECTED_TABLE_C_SC4, 18))
  np.testing.assert_array_equal(out["table_c"][1].cpu().numpy()[:, :18],
                                moved(EXPECTED_ACC_C_SC4, 18))
  for got, logical in zip(out["table_d"], (EXPECTED_TABLE_D, EXPECTED_ACC_D,
                                           EXPECTED_STEP_D)):
    np.testing.assert_allclose(
        got.cpu().numpy()[:, :8],
        _shard(np.tile(logical[:, None], (1, 8)), num_sc), rtol=1e-5,
        atol=1e-5)


def test_validation_mode_checks_the_forward_and_backward():
  """With validation on, the embedding API's lookup and update read back the
  kernels' status word: clean calls pass, and a sample view mislabelled as
  repeating no activation row (three ids per sample, so a row's entries
  straddle positions 255 and 256) raises instead of returning wrong
  activations silently."""
  from jax_tpu_embedding.sparsecore import _native  # pylint: disable=g-import-not-at-top

  table = embedding_spec.TableSpec(
      vocabulary_size=4096, embedding_dim=16, initializer=None,
      optimizer=embedding_spec.SGDOptimizerSpec(0.01), combiner="sum",
      name="t", max_ids_per_partition=4096,
      max_unique_ids_per_partition=4096)
  feature = embedding_spec.FeatureSpec(table_spec=table, input_shape=[512, 3],
                                       output_shape=[512, 16], name="f")
  embedding.prepare_feature_specs_for_training([feature], 1, 1)
  ids = np.stack([np.arange(512) * 3 + k for k in range(3)],
                 axis=1).astype(np.int32) % 4096
  prev = _native.set_validation(True)
  try:
    pre, _ = embedding.preprocess_sparse_dense_matmul_input(
        [ids], None, [feature], 1, 1, num_sc_per_device=1)
    variables = {"t": embedding.EmbeddingVariables(
        table=_cuda(_row_table(4096, 16)), slot=())}
    acts = embedding.tpu_sparse_dense_matmul(pre, variables, [feature],
                                             global_device_count=1,
                                             num_sc_per_device=1)
    np.testing.assert_array_equal(
        acts[0].cpu().numpy()[:, 0], ids.astype(np.float32).sum(axis=1))
    embedding.tpu_sparse_dense_matmul_grad(
        [torch.ones(512, 16).cuda()], pre, variables, [feature],
        num_sc_per_device=1)
    views = getattr(pre, "lookup_views", None)
    if not views:
      pytest.skip("the preprocessing built no lookup view")
    v = views["t"]
    views["t"] = _native.LookupView(v.keys, v.entries, v.device_batch_size,
                                    v.table_rows, v.num_entries,
                                    one_entry_per_key=True)
    with pytest.raises(RuntimeError, match="repeats a row"):
      embedding.tpu_sparse_dense_matmul(pre, variables, [feature],
                                        global_device_count=1,
                                        num_sc_per_device=1)
  finally:
    _native.set_validation(prev)
