"""Known-answer tests of the optimizers with two slot variables, transcribed
from the reference's primitive tests (lib/core/primitives/tests/):

  Adam      sparse_dense_matmul_grad_with_adam_test.py:403-411 (expectation:
            textbook Adam with bias-corrected m_hat / v_hat), :443-588 (ids,
            table row i = i + 1, momentum 0.002, velocity 0.004, grad 0.012,
            lr 0.1, beta 0.9 / 0.999, eps 1e-8; alpha_t and epsilon_hat as
            the test derives them; clipping to [2, 10])
  AdagradMomentum  sparse_dense_matmul_grad_with_adagrad_momentum_test.py:
            274-317 (expectation), :319-482 (accumulator 0.002, momentum
            0.004, lr 0.1, momentum 0.9, beta2 0.999, eps 1e-8, exponent
            -0.5, no Nesterov; clipping to [2, 12])
  FTRL      sparse_dense_matmul_grad_with_ftrl_test.py:235-321 (expectation:
            the sign / threshold form of the proximal step), :347-507
            (accumulator 0.002, linear 0.004, lr 0.1, lr_power -0.05, l1 2,
            l2 3, beta 0.5; clipping to [2, 12])
  LaProp    sparse_dense_matmul_grad_with_laprop_test.py:414-562 (table row
            i = i, mu 0.002, nu 0.004, grad 0.01, lr 0.1, b1 0.9, decay 0.95,
            eps 1e-8; clipping to [2, 12])
  F2A       sparse_dense_matmul_grad_with_f2a_test.py:500-722 (16 samples of
            4 ids, every id twice; table = arange, accumulator 0.1, local
            step 0, grad 0.1, lr 0.01, rho 1, global step 100, l1 = l2 = 0.01,
            max multiplier 10; clipping to [2, 12])

Each case runs on the CPU oracle and, marked gpu, through the product's
primitives, for 1, 2 and 4 SparseCores per device, with the reference's
tolerance (atol 1e-5). The expectations are the reference tests' own numpy
formulas, evaluated in float64.

Besides the transcribed cases, closed forms pin the oracle where the KATs
leave freedom (each would fail on a dropped term, a wrong sign or a swapped
operand):
  * FTRL with l1 = l2 = beta = 0, lr_power = -1/2 and the linear slot at
    -table * sqrt(accumulator) / lr is exactly Adagrad (the FTRL-proximal /
    Adagrad equivalence);
  * F2A with rho = 0 and no regularisation is Adagrad, and its local step
    counts the updates;
  * AdagradMomentum with momentum 0, beta2 = 1, exponent 2, eps 0 is Adagrad;
  * Adam's first step from zero slots moves each value by lr * g / (|g| +
    eps), so by about -lr * sign(g);
  * LaProp with the bias-corrected decay of LaPropOptimizerSpec keeps nu at
    g^2 + eps for a constant gradient over several steps, and its first step
    from zero slots is sqrt(1 - b1^2) * g / sqrt(g^2 + eps).
"""

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore.lib.core import input_preprocessing
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from jax_tpu_embedding.sparsecore.utils import utils
from oracle import refcpu

IDS = np.array([5, 3, 9, 1, 6, 12, 0, 4, 15, 13, 11, 7, 8, 14, 2, 10],
               np.int32).reshape(16, 1)
F2A_IDS = np.concatenate([np.arange(32, dtype=np.int32).reshape(8, 4)] * 2)
VOCAB, DIM, BATCH = 32, 8, 16
NUM_SCS = [1, 2, 4]


def _table_grad(ids, grad_value):
  """Dense table gradient of the reference tests' _compute_table_grad:
  every id of every sample adds weight 1 * grad."""
  g = np.zeros((VOCAB, DIM), np.float64)
  for row in ids:
    for i in row:
      g[i] += grad_value
  return g


def _f64(x):
  return np.asarray(x, np.float64)


def _expected_adam(g, t, m, v):
  """adam_test.py:403-411 (textbook Adam, t = 0 -> 1)."""
  lr, b1, b2, eps = 0.1, 0.9, 0.999, 1e-8
  m = b1 * m + (1 - b1) * g
  v = b2 * v + (1 - b2) * (g * g)
  m_hat = m / (1 - b1)
  v_hat = v / (1 - b2)
  return t - (lr * m_hat) / (np.sqrt(v_hat) + eps), m, v


def _expected_adagrad_momentum(g, e, a, m):
  """adagrad_momentum_test.py:274-317."""
  lr, mom, beta2, eps, k = 0.1, 0.9, 0.999, 1e-8, -0.5
  a_n = beta2 * a + (1.0 - beta2) * (g * g)
  g_hat = np.power(a_n + eps, -1.0 / k) * g
  m_n = mom * m + g_hat
  return e - lr * m_n, a_n, m_n


def _expected_ftrl(g, e, a, lin):
  """ftrl_test.py:235-321 (multiply_linear_by_learning_rate False)."""
  lr, lr_power, l1, l2, beta = 0.1, -0.05, 2.0, 3.0, 0.5
  a_new = a + g * g
  delta_p = np.power(a_new, -lr_power) - np.power(a, -lr_power)
  lin_new = lin + g - (delta_p / lr) * e
  numerator = np.sign(lin_new) * l1 - lin_new
  denominator = (np.power(a_new, -lr_power) + beta) / lr + 2 * l2
  w = np.where(np.abs(lin_new) > l1, numerator / denominator, 0.0)
  return w, a_new, lin_new


def _expected_laprop(g, theta, mu, nu):
  """laprop_test.py:483-489."""
  alpha, b1, decay, eps = 0.1, 0.9, 0.95, 1e-8
  nu_new = decay * nu + (1.0 - decay) * (g * g + eps)
  mu_new = b1 * mu + np.sqrt(1.0 - b1 ** 2) * (g / np.sqrt(nu_new))
  return theta - alpha * mu_new, mu_new, nu_new


def _expected_f2a(g, theta, a, l_step):
  """f2a_test.py:589-620."""
  alpha, rho, l1, l2, max_mult, g_step = 0.01, 1.0, 0.01, 0.01, 10.0, 100.0
  l_step_new = l_step + 1.0
  fa = np.minimum(np.power(max(g_step, 1.0) / l_step_new, rho), max_mult)
  a_new = a + g * g
  update = (fa * g) / np.sqrt(a_new) + l1 * np.sign(theta) + l2 * theta
  return theta - alpha * update, a_new, l_step_new


def _adam_hyper():
  # adam_test.py:541-543: alpha_t and epsilon_hat at step 0.
  c_2 = np.sqrt(np.float32(1.0) - np.float32(0.999))
  return (np.float32(0.1) * c_2 / (np.float32(1.0) - np.float32(0.9)),
          np.float32(0.9), np.float32(0.999), np.float32(1e-8) * c_2)


CASES = {
    "adam": dict(
        ids=IDS, grad=0.012, table=lambda: np.arange(VOCAB)[:, None] + 1.0,
        slots=(0.002, 0.004), hyper=_adam_hyper, expected=_expected_adam,
        clip=(2.0, 10.0), flags={}),
    "adagrad_momentum": dict(
        ids=IDS, grad=0.012, table=lambda: np.arange(VOCAB)[:, None] + 1.0,
        slots=(0.002, 0.004),
        hyper=lambda: (np.float32(0.1), np.float32(0.9), np.float32(0.999),
                       np.float32(1e-8), np.float32(-0.5), np.bool_(False)),
        expected=_expected_adagrad_momentum, clip=(2.0, 12.0), flags={}),
    "ftrl": dict(
        ids=IDS, grad=0.012, table=lambda: np.arange(VOCAB)[:, None] + 1.0,
        slots=(0.002, 0.004),
        hyper=lambda: (np.float32(0.1), np.float32(-0.05), np.float32(2.0),
                       np.float32(3.0), np.float32(0.5)),
        expected=_expected_ftrl, clip=(2.0, 12.0),
        flags={"multiply_linear_by_learning_rate": False}),
    "laprop": dict(
        ids=IDS, grad=0.01, table=lambda: np.arange(VOCAB)[:, None] + 0.0,
        slots=(0.002, 0.004),
        hyper=lambda: (np.float32(0.1), np.float32(0.9), 0.95,
                       np.float32(1e-8)),
        expected=_expected_laprop, clip=(2.0, 12.0), flags={}),
    "f2a": dict(
        ids=F2A_IDS, grad=0.1,
        table=lambda: np.arange(VOCAB * DIM).reshape(VOCAB, DIM),
        slots=(0.1, 0.0),
        hyper=lambda: (0.01, 1.0, 0.01, 0.01, 10.0, 100.0),
        expected=_expected_f2a, clip=(2.0, 12.0), flags={}),
}


def _case_arrays(name):
  c = CASES[name]
  table = np.ascontiguousarray(
      np.broadcast_to(c["table"](), (VOCAB, DIM)), np.float32)
  slots = [np.full((VOCAB, DIM), v, np.float32) for v in c["slots"]]
  return c, table, slots


def _expectation(name, lo, hi):
  c, table, slots = _case_arrays(name)
  g = _table_grad(c["ids"], c["grad"])
  t_new, s0, s1 = c["expected"](g, _f64(table), _f64(slots[0]),
                                _f64(slots[1]))
  touched = np.zeros(VOCAB, bool)
  touched[np.unique(c["ids"])] = True
  if lo is not None:
    t_new = np.clip(t_new, lo, hi)
  exp = [np.where(touched[:, None], t_new, table),
         np.where(touched[:, None], s0, slots[0]),
         np.where(touched[:, None], s1, slots[1])]
  return table, slots, exp


def _oracle_csr(ids, num_sc):
  max_ids = 64 // num_sc
  fs = input_preprocessing.single_feature_spec(
      ids.shape[0], VOCAB - 1, max_ids, 64, ids.shape[1], num_sc)
  r = refcpu.preprocess([ids], [np.ones_like(ids, np.float32)], [fs], 1, 1,
                        num_sc_per_device=num_sc)
  name = fs.table_spec.stacked_table_spec.stack_name
  return (r.row_pointers[name], r.embedding_ids[name], r.sample_ids[name],
          r.gains[name])


def _shard(table, num_sc):
  return np.ascontiguousarray(
      utils.shard_emb_table(table, num_devices=1, num_sc_per_device=num_sc)[0])


def _unshard(table, num_sc):
  return utils.unshard_emb_table(np.asarray(table)[np.newaxis],
                                 num_sc_per_device=num_sc)


CLIPS = [(None, None), "case"]


def _bounds(name, clip):
  return (None, None) if clip != "case" else CASES[name]["clip"]


@pytest.mark.parametrize("num_sc", NUM_SCS)
@pytest.mark.parametrize("clip", CLIPS)
@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_optimizer_kat(name, clip, num_sc):
  lo, hi = _bounds(name, clip)
  c = CASES[name]
  table, slots, exp = _expectation(name, lo, hi)
  grad = np.full((c["ids"].shape[0], DIM), c["grad"], np.float32)
  got = refcpu.sparse_dense_matmul_grad_optimizer(
      *_oracle_csr(c["ids"], num_sc), grad, _shard(table, num_sc),
      [_shard(s, num_sc) for s in slots], optimizer=name,
      hyperparameters=c["hyper"](), num_sc_per_device=num_sc, num_scs=num_sc,
      multiply_linear_by_lr=bool(
          c["flags"].get("multiply_linear_by_learning_rate", False)),
      min_value=lo, max_value=hi)
  for g, e, what in zip(got, exp, ("table", "slot 0", "slot 1")):
    np.testing.assert_allclose(_unshard(g, num_sc), e, atol=1e-5,
                               err_msg=f"{name} {what}")


# ---------------------------------------------------------------------------
# Closed forms.
# ---------------------------------------------------------------------------


def _random_case(seed, batch=64, vocab=48, dim=8, ids_per_row=3):
  rng = np.random.default_rng(seed)
  ids = rng.integers(0, vocab, size=(batch, ids_per_row)).astype(np.int32)
  fs = input_preprocessing.single_feature_spec(batch, vocab - 1, 4096, 4096,
                                               ids_per_row, 1)
  r = refcpu.preprocess([ids], [np.ones_like(ids, np.float32)], [fs], 1, 1,
                        num_sc_per_device=1)
  name = fs.table_spec.stacked_table_spec.stack_name
  csr = (r.row_pointers[name], r.embedding_ids[name], r.sample_ids[name],
         r.gains[name])
  table = rng.normal(0.0, 1.0, size=(vocab, dim)).astype(np.float32)
  grad = rng.normal(0.0, 1.0, size=(batch, dim)).astype(np.float32)
  touched = np.zeros(vocab, bool)
  touched[np.unique(ids)] = True
  return csr, table, grad, touched, rng


def _run(csr, grad, table, slots, optimizer, hyper, **kw):
  return refcpu.sparse_dense_matmul_grad_optimizer(
      *csr, grad, table, slots, optimizer=optimizer, hyperparameters=hyper,
      num_sc_per_device=1, num_scs=1, **kw)


def test_oracle_ftrl_reduces_to_adagrad():
  csr, table, grad, touched, _ = _random_case(1)
  acc = np.full(table.shape, 0.5, np.float32)
  lr = np.float32(0.05)
  lin = (-table.astype(np.float64) * np.sqrt(0.5) / lr).astype(np.float32)
  ftrl_t, ftrl_a, _ = _run(csr, grad, table, [acc, lin], "ftrl",
                           (lr, -0.5, 0.0, 0.0, 0.0))
  ada_t, ada_a = _run(csr, grad, table, [acc], "adagrad", (lr,))
  np.testing.assert_array_equal(ftrl_a, ada_a)
  np.testing.assert_allclose(ftrl_t, ada_t, rtol=2e-5, atol=2e-5)
  assert not np.allclose(ada_t[touched], table[touched])


def test_oracle_f2a_reduces_to_adagrad():
  csr, table, grad, touched, _ = _random_case(2)
  acc = np.full(table.shape, 0.1, np.float32)
  steps = np.full(table.shape, 3.0, np.float32)
  f2a_t, f2a_a, f2a_s = _run(csr, grad, table, [acc, steps], "f2a",
                             (0.01, 0.0, 0.0, 0.0, 1e6, 100.0))
  ada_t, ada_a = _run(csr, grad, table, [acc], "adagrad", (0.01,))
  np.testing.assert_array_equal(f2a_a, ada_a)
  np.testing.assert_allclose(f2a_t, ada_t, rtol=1e-6, atol=1e-7)
  np.testing.assert_array_equal(f2a_s[touched], 4.0)
  np.testing.assert_array_equal(f2a_s[~touched], 3.0)


def test_oracle_f2a_frequency_multiplier_and_regularisation():
  """fa = min((global_step / local_step)^rho, max) and the l1 / l2 terms,
  against a float64 evaluation of the reference test's formula on one
  entry per row (the summed gradient is then exact)."""
  rng = np.random.default_rng(3)
  vocab, dim, batch = 16, 4, 16
  ids = rng.permutation(vocab)[:batch].astype(np.int32).reshape(batch, 1)
  fs = input_preprocessing.single_feature_spec(batch, vocab - 1, 4096, 4096,
                                               1, 1)
  r = refcpu.preprocess([ids], [np.ones_like(ids, np.float32)], [fs], 1, 1,
                        num_sc_per_device=1)
  name = fs.table_spec.stacked_table_spec.stack_name
  csr = (r.row_pointers[name], r.embedding_ids[name], r.sample_ids[name],
         r.gains[name])
  table = rng.normal(0.0, 1.0, size=(vocab, dim)).astype(np.float32)
  table[0, 0] = 0.0  # sign(0) = 0
  grad = rng.normal(0.0, 1.0, size=(batch, dim)).astype(np.float32)
  acc = np.full(table.shape, 0.1, np.float32)
  steps = rng.integers(0, 50, size=table.shape).astype(np.float32)
  got_t, _, _ = _run(csr, grad, table, [acc, steps], "f2a",
                     (0.01, 0.5, 0.02, 0.03, 4.0, 40.0))
  g = np.zeros(table.shape)
  g[ids[:, 0]] = grad
  fa = np.minimum(np.power(40.0 / (_f64(steps) + 1.0), 0.5), 4.0)
  upd = (g * fa) / np.sqrt(0.1 + g * g) + 0.02 * np.sign(table) + 0.03 * table
  np.testing.assert_allclose(got_t, table - 0.01 * upd, rtol=1e-5, atol=1e-6)


def test_oracle_adagrad_momentum_reduces_to_adagrad():
  csr, table, grad, _, _ = _random_case(4)
  acc = np.full(table.shape, 0.2, np.float32)
  mom = np.zeros(table.shape, np.float32)
  am_t, am_a, am_m = _run(csr, grad, table, [acc, mom], "adagrad_momentum",
                          (0.03, 0.0, 1.0, 0.0, 2.0, False))
  ada_t, ada_a = _run(csr, grad, table, [acc], "adagrad", (0.03,))
  np.testing.assert_array_equal(am_a, ada_a)
  np.testing.assert_allclose(am_t, ada_t, rtol=1e-6, atol=1e-6)
  # With nesterov and momentum k the step is lr * (k * m + s), m = k m0 + s.
  m0 = np.full(table.shape, 0.25, np.float32)
  nt, _, nm = _run(csr, grad, table, [acc, m0], "adagrad_momentum",
                   (0.03, 0.5, 1.0, 0.0, 2.0, True))
  _, _, plain_m = _run(csr, grad, table, [acc, m0], "adagrad_momentum",
                       (0.03, 0.5, 1.0, 0.0, 2.0, False))
  np.testing.assert_array_equal(nm, plain_m)
  s = _f64(plain_m) - 0.5 * 0.25
  np.testing.assert_allclose(nt, table - 0.03 * (0.5 * _f64(plain_m) + s),
                             rtol=1e-5, atol=1e-6)


def test_oracle_adam_first_step_is_sign_step():
  csr, table, grad, touched, _ = _random_case(5)
  spec = embedding_spec.AdamOptimizerSpec(learning_rate=0.01)
  hyper = spec.get_hyperparameters(0)
  z = np.zeros(table.shape, np.float32)
  got_t, got_m, got_v = _run(csr, grad, table, [z, z], "adam", hyper)
  step = table - got_t
  g = got_m / np.float32(0.1)  # m = (1 - beta_1) * g
  np.testing.assert_allclose(got_v[touched], (0.001 * g * g)[touched],
                             rtol=1e-4)
  exp = 0.01 * g / (np.abs(g) + 1e-8)
  np.testing.assert_allclose(step[touched], exp[touched], rtol=1e-3,
                             atol=1e-6)
  np.testing.assert_array_equal(step[~touched], 0.0)


def test_oracle_laprop_bias_corrected_decay():
  """get_decay_rate(step) makes nu the plain average of g^2 + eps: with a
  constant gradient it stays g^2 + eps; the first step from zero slots is
  sqrt(1 - b1^2) g / sqrt(g^2 + eps)."""
  csr, table, grad, touched, _ = _random_case(6, ids_per_row=1, batch=32,
                                              vocab=64)
  spec = embedding_spec.LaPropOptimizerSpec(learning_rate=0.02, b1=0.8,
                                            b2=0.9, eps=1e-6)
  mu = np.zeros(table.shape, np.float32)
  nu = np.zeros(table.shape, np.float32)
  t = table
  for step in range(3):
    t, mu, nu = _run(csr, grad, t, [mu, nu], "laprop",
                     spec.get_hyperparameters(step))
    if step == 0:
      g = np.zeros(table.shape)
      np.add.at(g, csr[1][:int(csr[0][-1])], grad[csr[2][:int(csr[0][-1])]])
      exp_mu = np.sqrt(1 - 0.8 ** 2) * g / np.sqrt(g * g + 1e-6)
      np.testing.assert_allclose(mu[touched], exp_mu[touched], rtol=1e-5,
                                 atol=1e-6)
      g2 = g * g + 1e-6
  np.testing.assert_allclose(nu[touched], g2[touched], rtol=1e-5)
  np.testing.assert_array_equal(nu[~touched], 0.0)


def test_adam_hyperparameters_match_the_reference_derivation():
  """AdamOptimizerSpec.get_hyperparameters (embedding_spec.py:506-539)."""
  spec = embedding_spec.AdamOptimizerSpec(learning_rate=0.1)
  a, b1, b2, e = spec.get_hyperparameters(4)
  c2 = np.sqrt(1 - 0.999 ** 5)
  # float32 like the reference: 1 - 0.999^5 loses about 8 bits.
  np.testing.assert_allclose(a, 0.1 * c2 / (1 - 0.9 ** 5), rtol=5e-5)
  np.testing.assert_allclose(e, 1e-8 * c2, rtol=5e-5)
  assert b1.dtype == np.float32 and a.dtype == np.float32


def test_laprop_rejects_rms_clip_threshold():
  with pytest.raises(ValueError, match="rms_clip_threshold"):
    embedding_spec.LaPropOptimizerSpec(rms_clip_threshold=1.0)


# ---------------------------------------------------------------------------
# GPU: the product primitives on the same cases.
# ---------------------------------------------------------------------------


def _gpu():
  torch = pytest.importorskip("torch")
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  return torch


def _primitive(name):
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad_momentum as am  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adam as adam  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_f2a as f2a  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_ftrl as ftrl  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_laprop as laprop  # pylint: disable=g-import-not-at-top

  return {
      "adam": adam.tpu_sparse_dense_matmul_grad_with_adam_primitive,
      "adagrad_momentum": (
          am.tpu_sparse_dense_matmul_grad_with_adagrad_momentum_primitive),
      "ftrl": ftrl.tpu_sparse_dense_matmul_grad_with_ftrl_primitive,
      "laprop": laprop.tpu_sparse_dense_matmul_grad_with_laprop_primitive,
      "f2a": f2a.tpu_sparse_dense_matmul_grad_with_f2a_primitive,
  }[name]


@pytest.mark.gpu
@pytest.mark.parametrize("num_sc", NUM_SCS)
@pytest.mark.parametrize("clip", CLIPS)
@pytest.mark.parametrize("name", sorted(CASES))
def test_gpu_optimizer_kat(name, clip, num_sc):
  torch = _gpu()
  lo, hi = _bounds(name, clip)
  c = CASES[name]
  table, slots, exp = _expectation(name, lo, hi)
  ids = c["ids"]
  csr = input_preprocessing.preprocess_sparse_dense_matmul_input(
      ids, np.ones_like(ids, np.float32), 1,
      max_ids_per_partition=64 // num_sc, max_unique_ids_per_partition=64,
      num_sc_per_device=num_sc)
  grad = torch.full((ids.shape[0], DIM), c["grad"], dtype=torch.float32,
                    device="cuda")
  out = _primitive(name).bind(
      *csr, 1, torch.from_numpy(_shard(table, num_sc)).cuda(),
      *[torch.from_numpy(_shard(s, num_sc)).cuda() for s in slots], grad,
      *c["hyper"](), max_ids_per_partition=16,
      max_unique_ids_per_partition=16,
      computation_name="optimizer_test_computation", sharding_strategy=1,
      min_value=lo, max_value=hi, num_sc_per_device=num_sc, **c["flags"])
  assert len(out) == 3
  for g, e, what in zip(out, exp, ("table", "slot 0", "slot 1")):
    np.testing.assert_allclose(_unshard(g.cpu().numpy(), num_sc), e,
                               atol=1e-5, err_msg=f"{name} {what}")
