"""Custom optimizer updates on the GPU.

Transcribed from the reference (paths under jax_tpu_embedding/sparsecore/):
  lib/core/primitives/tests/sparse_dense_matmul_optimizer_grad_test.py
      :142-626: the primitive bound with SGD, Adagrad, FTRL, Adam and a
      clipped SGD as StableHLO update functions; the expectation is the
      function evaluated (here in numpy float32) on the touched rows with
      their summed gradients (`_get_expected_updated_table`, :81-140),
      compared with assert_allclose at its default rtol 1e-7 (the reference
      test's tolerance). The StableHLO comes from this build's
      `lower_to_stablehlo` (jax.jit(...).lower(...) in the reference), and for
      Adagrad also from text in jax's own form.
  lib/nn/tests/tpu_sparse_dense_matmul_grad_test.py:1324-1486
      (test_custom_optimizer_adagrad): the embedding API with a
      CustomOptimizerSpec; literal table and accumulator.
  lib/nn/tests/tpu_sparse_dense_matmul_grad_test.py:1488-1724
      (test_custom_optimizer_stacked): two tables stacked under a custom SGD
      and a custom Adagrad table; the reference's second device is left
      out (one GPU), its closed-form expectations kept.
Added here: custom SGD and Adagrad equal the built-in updates bit for bit on
multi-hot weighted input (the same kernel up to the update), and a random
custom update matches the oracle. Every test runs twice: with the programs
compiled for themselves at run time (SCEMB_CUSTOM_UPDATE=compile, where a
failure to compile fails the call) and interpreted; the two give identical
bits.
"""

import pathlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  torch.cuda.set_device(0)


@pytest.fixture(autouse=True, params=["compile", "interpret"])
def update_mode(request, monkeypatch):
  monkeypatch.setenv("SCEMB_CUSTOM_UPDATE", request.param)
  return request.param


from jax_tpu_embedding.sparsecore.lib.core import input_preprocessing  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as adagrad_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd as sgd_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_optimizer_grad as smog  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import custom_optimizer_lowering as col  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import table_stacking  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.utils import utils  # pylint: disable=g-import-not-at-top,wrong-import-position
from oracle import refcpu  # pylint: disable=g-import-not-at-top,wrong-import-position

# Adagrad's update as jax.jit(...).lower(...).as_text() writes it.
JAX_ADAGRAD = (pathlib.Path(__file__).parent / "golden" /
               "custom_adagrad_jax.stablehlo").read_text()

IDS = np.array([5, 3, 9, 1, 6, 12, 0, 4, 15, 13, 11, 7, 8, 14, 2, 10],
               np.int32).reshape(16, 1)
VOCAB, DIM, BATCH = 32, 8, 16


def _shard(table, num_sc):
  return np.ascontiguousarray(
      utils.shard_emb_table(table, num_devices=1, num_sc_per_device=num_sc)[0])


def _cuda(x):
  return torch.tensor(np.ascontiguousarray(x, np.float32)).cuda()


def _expected(emb_table, z_grad, indices, weights, fn, num_sc, *rest):
  """sparse_dense_matmul_optimizer_grad_test.py:81-140 in numpy: gradients
  summed per id, `fn` on the touched rows, the results sharded."""
  grad_full = np.zeros_like(emb_table)
  np.add.at(grad_full, indices[:, 0], weights * z_grad)
  rows = np.unique(indices[:, 0])
  arrays = [i for i, a in enumerate(rest)
            if isinstance(a, np.ndarray) and a.shape == emb_table.shape]
  args = [a[rows] if i in arrays else a for i, a in enumerate(rest)]
  out = fn(grad_full[rows], emb_table[rows], *args)
  outs = out if isinstance(out, tuple) else (out,)
  result = [emb_table.copy()] + [rest[i].copy() for i in arrays]
  for r, o in zip(result, outs):
    r[rows] = o
  return tuple(_shard(r, num_sc) for r in result)


def _sgd(grad, table, lr):
  return table - lr * grad


def _adagrad(grad, table, accum, lr):
  new_accum = accum + grad * grad
  return table - lr * grad / np.sqrt(new_accum), new_accum


def _ftrl(grad, table, accum, linear, lr, lr_power, l1, l2, beta):
  two = np.float32(2.0)
  zero = np.float32(0.0)
  a_new = accum + grad * grad
  p_old = np.power(accum, -lr_power)
  p_new = np.power(a_new, -lr_power)
  delta_p = p_new - p_old
  new_linear = linear + grad - (delta_p / lr) * table
  l_threshold = l1
  numerator = np.sign(new_linear) * l_threshold - new_linear
  abs_l_new = np.abs(new_linear)
  denominator = (p_new + beta) / lr + two * l2
  w_new = np.where(abs_l_new > l_threshold, numerator / denominator, zero)
  return w_new, a_new, new_linear


def _adam(grad, table, m, v, alpha_t, beta_1, beta_2, epsilon_hat):
  new_m = beta_1 * m + (1.0 - beta_1) * grad
  new_v = beta_2 * v + (1.0 - beta_2) * (grad * grad)
  new_table = table - alpha_t * new_m / (np.sqrt(new_v) + epsilon_hat)
  return new_table, new_m, new_v


def _sgd_with_clip(grad, table, lr):
  return np.clip(_sgd(grad, table, lr), -2.0, 5.0)


def _emb_table():
  return np.repeat(np.arange(VOCAB, dtype=np.float32)[:, None], DIM, axis=1)


def _adam_hyper():
  lr, beta_1, beta_2, epsilon = 0.1, 0.9, 0.999, 1e-8
  c_2 = np.sqrt(1.0 - beta_2)
  return [lr * c_2 / (1.0 - beta_1), beta_1, beta_2, epsilon * c_2]


# (function, slot initial values, hyperparameters, gradient value)
PRIMITIVE_CASES = {
    "sgd": (_sgd, (), [0.01], 0.01),
    "adagrad": (_adagrad, (0.0,), [0.01], 0.01),
    "ftrl": (_ftrl, (0.1, 0.01), [0.1, -0.5, 0.001, 0.002, 0.01], 0.01),
    "adam": (_adam, (0.002, 0.004), _adam_hyper(), 0.01),
    "clipping": (_sgd_with_clip, (), [1.0], 10.0),
}


@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("case", list(PRIMITIVE_CASES))
def test_primitive_backward_pass(case, num_sc):
  """sparse_dense_matmul_optimizer_grad_test.py:142-626."""
  fn, slot_values, hyper, gval = PRIMITIVE_CASES[case]
  weights = np.ones_like(IDS, np.float32)
  csr = input_preprocessing.preprocess_sparse_dense_matmul_input(
      IDS, weights, 1, max_ids_per_partition=16,
      max_unique_ids_per_partition=64, num_sc_per_device=num_sc)
  table = _emb_table()
  slots = [np.full_like(table, v, np.float32) for v in slot_values]
  z_grad = np.full((BATCH, DIM), gval, np.float32)
  stablehlo = col.lower_to_stablehlo(fn, DIM, len(slots), len(hyper))
  got = smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
      *csr, np.int32(1), _cuda(z_grad), *hyper,
      *[_cuda(_shard(v, num_sc)) for v in (table, *slots)],
      num_hyperparameters=len(hyper), stablehlo=stablehlo,
      max_ids_per_partition=16, max_unique_ids_per_partition=16,
      computation_name="optimizer_test_computation", sharding_strategy=1,
      num_sc_per_device=num_sc)
  want = _expected(table, z_grad, IDS, weights, fn, num_sc, *slots,
                   *[np.float32(h) for h in hyper])
  assert len(got) == len(want) == 1 + len(slots)
  for g, w in zip(got, want):
    np.testing.assert_allclose(g.cpu().numpy(), w)


@pytest.mark.parametrize("num_sc", [1, 4])
def test_primitive_reads_jax_stablehlo_text(num_sc):
  """The Adagrad case with the update given as jax writes it."""
  csr = input_preprocessing.preprocess_sparse_dense_matmul_input(
      IDS, np.ones_like(IDS, np.float32), 1, max_ids_per_partition=16,
      max_unique_ids_per_partition=64, num_sc_per_device=num_sc)
  table = _emb_table()
  z_grad = np.full((BATCH, DIM), 0.01, np.float32)
  outs = []
  for text in (JAX_ADAGRAD, JAX_ADAGRAD.encode(),
               col.lower_to_stablehlo(_adagrad, DIM, 1, 1)):
    outs.append(smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
        *csr, np.int32(1), _cuda(z_grad), np.float32(0.01),
        _cuda(_shard(table, num_sc)), _cuda(np.zeros((VOCAB, DIM))),
        num_hyperparameters=1, stablehlo=text, max_ids_per_partition=16,
        max_unique_ids_per_partition=16, num_sc_per_device=num_sc))
  for t, a in outs[1:]:
    torch.testing.assert_close(t, outs[0][0], rtol=0, atol=0)
    torch.testing.assert_close(a, outs[0][1], rtol=0, atol=0)
  want = _expected(table, z_grad, IDS, np.ones_like(IDS, np.float32),
                   _adagrad, num_sc, np.zeros_like(table), np.float32(0.01))
  for g, w in zip(outs[0], want):
    np.testing.assert_allclose(g.cpu().numpy(), w)


def test_primitive_validates_operands():
  csr = input_preprocessing.preprocess_sparse_dense_matmul_input(
      IDS, np.ones_like(IDS, np.float32), 1, max_ids_per_partition=16,
      max_unique_ids_per_partition=64, num_sc_per_device=4)
  table = _cuda(_emb_table())
  grad = _cuda(np.ones((BATCH, DIM)))
  text = col.lower_to_stablehlo(_sgd, DIM, 0, 1)
  bind = smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind
  common = dict(max_ids_per_partition=16, max_unique_ids_per_partition=16,
                num_sc_per_device=4)
  with pytest.raises(ValueError, match="At least one embedding variable"):
    bind(*csr, np.int32(1), grad, np.float32(0.1), num_hyperparameters=1,
         stablehlo=text, **common)
  with pytest.raises(ValueError, match="hyperparameters must be float32"):
    bind(*csr, np.int32(1), grad, np.int32(1), table, num_hyperparameters=1,
         stablehlo=text, **common)
  with pytest.raises(ValueError, match="scalars or 1D of size 1"):
    bind(*csr, np.int32(1), grad, np.zeros(2, np.float32), table,
         num_hyperparameters=1, stablehlo=text, **common)
  with pytest.raises(ValueError, match="stablehlo must be a string"):
    bind(*csr, np.int32(1), grad, np.float32(0.1), table,
         num_hyperparameters=1, stablehlo=None, **common)
  with pytest.raises(ValueError, match="@main takes 3 arguments"):
    bind(*csr, np.int32(1), grad, np.float32(0.1), table, table.clone(),
         num_hyperparameters=1, stablehlo=text, **common)


# --- tpu_sparse_dense_matmul_grad_test.py:1324-1486 --------------------------

EXPECTED_TABLE_C_SC4 = np.array(
    [-1.000e-02, 3.990e00, 7.990e00, 1.199e01, 1.600e01, 2.000e01, 2.400e01,
     2.800e01, 9.900e-01, 4.990e00, 8.990e00, 1.299e01, 1.700e01, 2.100e01,
     2.500e01, 2.900e01, 1.990e00, 5.990e00, 9.990e00, 1.399e01, 1.800e01,
     2.200e01, 2.600e01, 3.000e01, 2.990e00, 6.990e00, 1.099e01, 1.499e01,
     1.900e01, 2.300e01, 2.700e01, 3.100e01], np.float32)
EXPECTED_ACC_C_SC4 = np.array(([1.0] * 4 + [0.0] * 4) * 4, np.float32)


def _unshard4(values):
  out = np.empty_like(values)
  for r in range(32):
    out[r] = values[(r % 4) * 8 + r // 4]
  return out


@pytest.mark.parametrize("num_sc", [1, 2, 4])
def test_custom_optimizer_adagrad(num_sc):
  def adagrad_fn(grad, table, accum, lr):
    new_accum = accum + grad * grad
    return table - lr * grad / np.sqrt(new_accum), new_accum

  spec = embedding_spec.CustomOptimizerSpec(
      learning_rate=0.01, custom_computation_fn=adagrad_fn,
      slot_variable_initializers_tuple=(lambda *_: 0.0,),
      short_name_str="custom_adagrad")
  table_c = embedding_spec.TableSpec(
      vocabulary_size=32, embedding_dim=18, initializer=None, optimizer=spec,
      combiner="sum", name="table_c")
  feature_specs = {"feature_spec_c": embedding_spec.FeatureSpec(
      table_spec=table_c, input_shape=(16, 1), output_shape=(16, 18),
      name="feature_spec_c")}
  embedding.prepare_feature_specs_for_training(
      feature_specs, num_sc_per_device=num_sc, global_device_count=1)
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      {"feature_spec_c": IDS}, features_weights=None,
      feature_specs=feature_specs, local_device_count=1,
      global_device_count=1, num_sc_per_device=num_sc,
      sharding_strategy="MOD")
  logical = np.repeat(np.arange(32, dtype=np.float32)[:, None], 24, axis=1)
  variables = {"table_c": (_cuda(_shard(logical, num_sc)),
                           _cuda(np.zeros((32, 24))))}
  grads = {"feature_spec_c": torch.ones(16, 18).cuda()}
  out = embedding.tpu_sparse_dense_matmul_grad(
      grads, pre, variables, feature_specs, sharding_strategy="MOD",
      num_sc_per_device=num_sc)

  def moved(sc4_values):
    return _shard(np.repeat(_unshard4(sc4_values)[:, None], 18, axis=1),
                  num_sc)

  np.testing.assert_allclose(out["table_c"][0].cpu().numpy()[:, :18],
                             moved(EXPECTED_TABLE_C_SC4))
  np.testing.assert_allclose(out["table_c"][1].cpu().numpy()[:, :18],
                             moved(EXPECTED_ACC_C_SC4))


# --- tpu_sparse_dense_matmul_grad_test.py:1488-1724 --------------------------

INPUT_A = np.array([np.array(r, np.int32) for r in (
    [5, 4, 2], [3], [9], [1, 9, 16], [6, 12, 1, 10], [12, 19],
    [0, 15, 2, 25, 25], [4, 28, 25], [15, 0], [13], [11], [7, 1], [8, 9],
    [14, 14, 14], [2, 28], [10, 16])], dtype=object)
INPUT_B = np.array([np.array(r, np.int32) for r in (
    [50, 40, 20], [33], [59], [1, 9, 16], [6, 12, 1, 10], [12, 19],
    [0, 15, 2, 25, 25], [4, 28, 25], [50, 51, 0], [10, 50, 60],
    [11, 12, 13], [61, 60], [58, 2], [41, 41, 50], [2, 58], [10, 16])],
                   dtype=object)


def _count(rows, v):
  return sum(int(x == v) for r in rows for x in r)


def test_custom_optimizer_stacked():
  def simple_sgd(grad, table, lr):
    return table - lr * grad

  def adagrad_fn(grad, table, accum, lr):
    new_accum = accum + grad * grad
    return table - lr * grad / (np.sqrt(new_accum) + 1e-7), new_accum

  custom_sgd = embedding_spec.CustomOptimizerSpec(
      learning_rate=0.01, custom_computation_fn=simple_sgd,
      short_name_str="custom_sgd")
  custom_adagrad = embedding_spec.CustomOptimizerSpec(
      learning_rate=0.01, custom_computation_fn=adagrad_fn,
      slot_variable_initializers_tuple=(lambda *_: 0.0,),
      short_name_str="custom_adagrad")

  def table(name, vocab, dim, opt):
    return embedding_spec.TableSpec(
        vocabulary_size=vocab, embedding_dim=dim, initializer=None,
        optimizer=opt, combiner="sum", name=name)

  tables = {"a": table("table_a", 32, 8, custom_sgd),
            "b": table("table_b", 64, 8, custom_sgd),
            "c": table("table_c", 32, 16, custom_adagrad)}
  feature_specs = {
      f"feature_spec_{k}": embedding_spec.FeatureSpec(
          table_spec=t, input_shape=(16, 1),
          output_shape=(16, t.embedding_dim), name=f"feature_spec_{k}")
      for k, t in tables.items()}
  embedding.auto_stack_tables(feature_specs, global_device_count=1,
                              num_sc_per_device=4)
  embedding.prepare_feature_specs_for_training(
      feature_specs, global_device_count=1, num_sc_per_device=4)
  specs = {k: feature_specs[f"feature_spec_{k}"].table_spec for k in tables}
  assert specs["a"].stacked_table_spec.stack_name == (
      specs["b"].stacked_table_spec.stack_name)
  inputs = {"feature_spec_a": INPUT_A, "feature_spec_b": INPUT_B,
            "feature_spec_c": IDS}
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      inputs, features_weights=None, feature_specs=feature_specs,
      local_device_count=1, global_device_count=1, num_sc_per_device=4,
      sharding_strategy="MOD", batch_number=42)

  vocabs = {"a": 32, "b": 64, "c": 32}
  offsets = {"a": 0, "b": 100, "c": 0}
  logical = {k: np.repeat((np.arange(vocabs[k]) + offsets[k]).astype(
      np.float32)[:, None], tables[k].embedding_dim, axis=1) for k in tables}
  stacked = table_stacking.stack_and_shard_tables(
      {k: specs[k] for k in tables}, logical, num_shards=4)
  names = {k: (specs[k].stacked_table_spec.stack_name
               if specs[k].is_stacked() else specs[k].name) for k in tables}
  ab, c = names["a"], names["c"]
  variables = {
      ab: (_cuda(stacked[ab].reshape(-1, stacked[ab].shape[-1])),),
      c: (_cuda(stacked[c].reshape(-1, stacked[c].shape[-1])),
          _cuda(np.zeros(stacked[c].reshape(-1, stacked[c].shape[-1]).shape))),
  }
  grads = {f"feature_spec_{k}": torch.ones(16, t.embedding_dim).cuda()
           for k, t in tables.items()}
  out = embedding.tpu_sparse_dense_matmul_grad(
      grads, pre, variables, feature_specs, sharding_strategy="MOD",
      num_sc_per_device=4)

  result = table_stacking.unshard_and_unstack_tables(
      {k: specs[k] for k in tables},
      {ab: out[ab][0].cpu().numpy(), c: out[c][0].cpu().numpy()},
      num_shards=4)
  for k, rows in (("a", INPUT_A), ("b", INPUT_B)):
    want = np.array([r + offsets[k] - np.float32(0.01) * _count(rows, r)
                     for r in range(vocabs[k])], np.float32)
    np.testing.assert_array_equal(
        result[k], np.repeat(want[:, None], 8, axis=1))
  counts = np.array([_count(IDS, r) for r in range(32)], np.float32)
  want_c = np.where(counts > 0,
                    np.arange(32) - 0.01 * counts / (counts + 1e-7),
                    np.arange(32)).astype(np.float32)
  np.testing.assert_allclose(result["c"], np.repeat(want_c[:, None], 16, 1),
                             rtol=1e-5, atol=1e-5)
  acc = table_stacking.unshard_and_unstack_tables(
      {"c": specs["c"]}, {c: out[c][1].cpu().numpy()}, num_shards=4)["c"]
  np.testing.assert_allclose(acc, np.repeat((counts ** 2)[:, None], 16, 1),
                             rtol=1e-5, atol=1e-5)


# --- against the built-in updates and the oracle ----------------------------

def _random_csr(num_sc, seed=5, batch=128, valency=7, vocab=256):
  rng = np.random.default_rng(seed)
  ids = rng.integers(0, vocab, size=(batch, valency)).astype(np.int32)
  weights = rng.uniform(0.25, 2.0, size=ids.shape).astype(np.float32)
  spec = input_preprocessing.single_feature_spec(batch, vocab - 1, 1024,
                                                 1024, 1, num_sc)
  r = refcpu.preprocess([ids], [weights], [spec], 1, 1,
                        num_sc_per_device=num_sc)
  n = spec.table_spec.stacked_table_spec.stack_name
  oracle_csr = (r.row_pointers[n], r.embedding_ids[n], r.sample_ids[n],
                r.gains[n])
  gpu_csr = input_preprocessing.preprocess_sparse_dense_matmul_input(
      ids, weights, 1, max_ids_per_partition=1024,
      max_unique_ids_per_partition=1024, num_sc_per_device=num_sc)
  return rng, oracle_csr, gpu_csr


@pytest.mark.parametrize("num_sc", [1, 4])
def test_custom_equals_builtin_sgd_and_adagrad(num_sc):
  rng, _, csr = _random_csr(num_sc)
  dim, rows = 16, 256
  table = rng.normal(size=(rows, dim)).astype(np.float32)
  acc = rng.uniform(0.1, 1.0, size=(rows, dim)).astype(np.float32)
  grad = _cuda(rng.normal(size=(128, dim)))
  common = dict(max_ids_per_partition=1024,
                max_unique_ids_per_partition=1024, num_sc_per_device=num_sc)

  (custom,) = smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
      *csr, np.int32(1), grad, np.float32(0.05), _cuda(table),
      num_hyperparameters=1, stablehlo=col.lower_to_stablehlo(_sgd, dim),
      **common)
  builtin = sgd_prim.tpu_sparse_dense_matmul_grad_with_sgd_primitive.bind(
      *csr, np.int32(1), _cuda(table), grad, np.float32(0.05), **common)
  torch.testing.assert_close(custom, builtin, rtol=0, atol=0)

  ct, ca = smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
      *csr, np.int32(1), grad, np.float32(0.05), _cuda(table), _cuda(acc),
      num_hyperparameters=1,
      stablehlo=col.lower_to_stablehlo(_adagrad, dim, 1, 1), **common)
  bt, ba = adagrad_prim.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
      *csr, np.int32(1), _cuda(table), _cuda(acc), grad, np.float32(0.05),
      **common)
  torch.testing.assert_close(ct, bt, rtol=0, atol=0)
  torch.testing.assert_close(ca, ba, rtol=0, atol=0)


def _mixed(grad, table, m, v, lr, decay):
  """Exercises most operations the kernel interprets."""
  new_m = np.maximum(decay * m, np.abs(grad))
  new_v = v + np.tanh(grad) * np.exp(-np.abs(grad)) + np.log1p(grad * grad)
  step = np.where(new_m > 0.5, grad / (np.sqrt(new_v * new_v) + 1e-6),
                  np.sign(grad) * np.minimum(np.abs(grad), 1.0))
  return np.clip(table - lr * step, -3.0, 3.0), new_m, new_v


@pytest.mark.parametrize("num_sc", [1, 4])
def test_custom_update_matches_oracle(num_sc):
  rng, ocsr, csr = _random_csr(num_sc, seed=9)
  dim, rows = 24, 256
  table = rng.normal(size=(rows, dim)).astype(np.float32)
  m = rng.uniform(0.0, 1.0, size=(rows, dim)).astype(np.float32)
  v = rng.uniform(0.0, 1.0, size=(rows, dim)).astype(np.float32)
  grad = rng.normal(size=(128, dim)).astype(np.float32)
  hyper = [np.float32(0.1), np.float32(0.9)]
  got = smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
      *csr, np.int32(1), _cuda(grad), *hyper, _cuda(table), _cuda(m),
      _cuda(v), num_hyperparameters=2,
      stablehlo=col.lower_to_stablehlo(_mixed, dim, 2, 2),
      max_ids_per_partition=1024, max_unique_ids_per_partition=1024,
      num_sc_per_device=num_sc)
  want = refcpu.sparse_dense_matmul_grad_custom(
      *ocsr, grad, table, [m, v], update_fn=_mixed, hyperparameters=hyper,
      num_sc_per_device=num_sc, num_scs=num_sc)
  # Gradient sums are added in another order on the GPU (a few ulp), and
  # exp / log1p / tanh are the device's own: 1e-5 relative, 1e-5 absolute.
  for g, w in zip(got, want):
    np.testing.assert_allclose(g.cpu().numpy(), w, rtol=1e-5, atol=1e-5)
  untouched = ~refcpu.touched_rows(ocsr[0], ocsr[1], num_sc_per_device=num_sc,
                                   num_scs=num_sc, table_rows=rows)
  np.testing.assert_array_equal(got[0].cpu().numpy()[untouched],
                                table[untouched])



def _arith(grad, table, m, v, lr, decay):
  """Arithmetic and comparison operations only, more than 8 registers."""
  new_m = np.maximum(decay * m, np.abs(grad))
  new_v = np.minimum(v + grad * grad, 4.0)
  step = np.where(new_m > 0.5, grad / (np.sqrt(new_v) + 1e-6), -grad)
  step = step + np.sign(table) * 0.01
  return np.clip(table - lr * step, -3.0, 3.0), new_m, new_v


@pytest.mark.parametrize("fn,dim", [(_adagrad, 16), (_arith, 16), (_mixed, 24),
                                    (_adagrad, 12)])
def test_compiled_equals_interpreted(fn, dim, monkeypatch):
  """Compiled and interpreted updates give the same bits (16-byte layout:
  Adagrad at dim 16; 4-byte layout: programs over 8 registers, programs with
  transcendental operations, dims that are not multiples of 4), both within
  the oracle's tolerance."""
  rng, ocsr, csr = _random_csr(4, seed=13)
  rows = 256
  table = rng.normal(size=(rows, dim)).astype(np.float32)
  m = rng.uniform(0.1, 1.0, size=(rows, dim)).astype(np.float32)
  v = rng.uniform(0.1, 1.0, size=(rows, dim)).astype(np.float32)
  grad = rng.normal(size=(128, dim)).astype(np.float32)
  if fn is _adagrad:
    slots, hyper = [m], [np.float32(0.1)]
  else:
    slots, hyper = [m, v], [np.float32(0.1), np.float32(0.9)]
  text = col.lower_to_stablehlo(fn, dim, len(slots), len(hyper))
  runs = {}
  for mode in ("compile", "interpret"):
    monkeypatch.setenv("SCEMB_CUSTOM_UPDATE", mode)
    runs[mode] = [
        x.cpu().numpy()
        for x in smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
            *csr, np.int32(1), _cuda(grad), *hyper, _cuda(table),
            *[_cuda(x) for x in slots], num_hyperparameters=len(hyper),
            stablehlo=text, max_ids_per_partition=1024,
            max_unique_ids_per_partition=1024, num_sc_per_device=4)]
  for c, i in zip(runs["compile"], runs["interpret"]):
    np.testing.assert_array_equal(c, i)
  want = refcpu.sparse_dense_matmul_grad_custom(
      *ocsr, grad, table, slots, update_fn=fn, hyperparameters=hyper,
      num_sc_per_device=4, num_scs=4)
  for g, w in zip(runs["compile"], want):
    np.testing.assert_allclose(g, w, rtol=1e-5, atol=1e-5)


def test_unknown_update_mode_is_an_error(monkeypatch):
  _, _, csr = _random_csr(1)
  monkeypatch.setenv("SCEMB_CUSTOM_UPDATE", "fast")
  with pytest.raises(ValueError, match="SCEMB_CUSTOM_UPDATE"):
    smog.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
        *csr, np.int32(1), _cuda(np.ones((128, 8))), np.float32(0.1),
        _cuda(np.zeros((256, 8))), num_hyperparameters=1,
        stablehlo=col.lower_to_stablehlo(_sgd, 8),
        max_ids_per_partition=1024, max_unique_ids_per_partition=1024,
        num_sc_per_device=1)
