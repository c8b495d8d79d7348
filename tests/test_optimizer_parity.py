"""GPU parity of the optimizers with two slot variables (Adam,
AdagradMomentum, FTRL, LaProp, F2A) against the CPU oracle
(oracle/refcpu.cc, ref_sparse_dense_matmul_grad_optimizer), through the
product primitives and the embedding API.

Tolerances: rtol 1e-5, atol 1e-6 (BASELINE's fp32 tolerance), with
  * one entry per touched row ("unique") or small-integer gradients on hot
    rows (Zipf ids, thousands of entries on a few rows: every partial sum is
    an exact integer), so the summed gradient is the same on both sides and
    only the rounding of the device and host sqrt / pow differs (the
    float summation order of hot rows is covered by test_gpu_parity, on the
    same reduction code);
  * FTRL's linear slot multiplies a difference of two powers by table / lr,
    so one ulp of a library pow is amplified: its bound adds that term
    (_ftrl_pow_bounds);
  * the in-place (CSR sorted by row) and sorting routes, dense and per-feature
    gradients, host and device hyperparameters, and repeated calls must agree
    bit for bit.
"""

import zlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  torch.cuda.set_device(0)


from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad_momentum as am_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adam as adam_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_f2a as f2a_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_ftrl as ftrl_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_laprop as laprop_prim  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import table_stacking  # pylint: disable=g-import-not-at-top,wrong-import-position
from oracle import refcpu  # pylint: disable=g-import-not-at-top,wrong-import-position

PRIMS = {
    "adam": adam_prim.tpu_sparse_dense_matmul_grad_with_adam_primitive,
    "adagrad_momentum": (
        am_prim.tpu_sparse_dense_matmul_grad_with_adagrad_momentum_primitive),
    "ftrl": ftrl_prim.tpu_sparse_dense_matmul_grad_with_ftrl_primitive,
    "ftrl_by_lr": ftrl_prim.tpu_sparse_dense_matmul_grad_with_ftrl_primitive,
    "laprop": laprop_prim.tpu_sparse_dense_matmul_grad_with_laprop_primitive,
    "f2a": f2a_prim.tpu_sparse_dense_matmul_grad_with_f2a_primitive,
}

HYPER = {
    "adam": (np.float32(0.004), np.float32(0.9), np.float32(0.999),
             np.float32(1e-7)),
    "adagrad_momentum": (np.float32(0.05), np.float32(0.8), np.float32(0.99),
                         np.float32(1e-6), np.float32(2.0), np.bool_(True)),
    "ftrl": (np.float32(0.05), np.float32(-0.5), np.float32(0.001),
             np.float32(0.002), np.float32(0.1)),
    "ftrl_by_lr": (np.float32(0.05), np.float32(-0.5), np.float32(0.001),
                   np.float32(0.002), np.float32(0.1)),
    "laprop": (np.float32(0.01), np.float32(0.9), np.float32(0.95),
               np.float32(1e-8)),
    "f2a": (np.float32(0.01), np.float32(0.5), np.float32(0.001),
            np.float32(0.002), np.float32(5.0), np.float32(100.0)),
}


def _oracle_name(name):
  return "ftrl" if name == "ftrl_by_lr" else name


def _flags(name):
  if name.startswith("ftrl"):
    return {"multiply_linear_by_learning_rate": name == "ftrl_by_lr"}
  return {}


def _slots(name, rng, shape):
  a = rng.normal(size=shape).astype(np.float32)
  b = rng.normal(size=shape).astype(np.float32)
  if name == "adam":
    return [0.01 * a, 0.01 * np.abs(b)]
  if name == "laprop":
    return [0.01 * a, 0.5 + 0.1 * np.abs(b)]
  if name == "f2a":
    return [0.1 + np.abs(a), np.floor(5 * np.abs(b))]
  return [0.1 + np.abs(a), 0.01 * b]  # accumulator + momentum / linear


def _zipf(rng, a, vocab, size):
  out = np.empty(size, np.int64)
  filled = 0
  while filled < size:
    k = rng.zipf(a, size=2 * (size - filled) + 16)
    k = k[k <= vocab]
    take = min(size - filled, len(k))
    out[filled:filled + take] = k[:take] - 1
    filled += take
  return out.astype(np.int32)


def _case(kind, rng, num_sc):
  """(features, feature spec, stack name, oracle preprocessing)."""
  if kind == "unique":
    batch, vocab, valency = 512, 2048, 1
    ids = rng.permutation(vocab)[:batch].astype(np.int32).reshape(batch, 1)
  else:
    batch, vocab, valency = 1024, 600, 8
    ids = _zipf(rng, 1.3, vocab, batch * valency).reshape(batch, valency)
  table = embedding_spec.TableSpec(
      name="t", vocabulary_size=vocab, embedding_dim=20,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.01), combiner="sum",
      max_ids_per_partition=1 << 16, max_unique_ids_per_partition=1 << 16)
  fs = embedding_spec.FeatureSpec(name="f", table_spec=table,
                                  input_shape=[batch, valency],
                                  output_shape=[batch, 20])
  embedding.prepare_feature_specs_for_training([fs], 1, num_sc)
  ref = refcpu.preprocess([ids], None, [fs], 1, 1, num_sc_per_device=num_sc)
  name = fs.table_spec.stacked_table_spec.stack_name
  return ids, fs, name, ref


def _bind(name, ref, sname, table, slots, grad, num_sc, hyper=None, **kw):
  return PRIMS[name].bind(
      ref.row_pointers[sname], ref.embedding_ids[sname],
      ref.sample_ids[sname], ref.gains[sname], 1, table, *slots, grad,
      *(hyper if hyper is not None else HYPER[name]),
      max_ids_per_partition=1 << 16, max_unique_ids_per_partition=1 << 16,
      num_sc_per_device=num_sc, **_flags(name), **kw)


def _oracle(name, ref, sname, table, slots, grad, num_sc, lo=None, hi=None):
  return refcpu.sparse_dense_matmul_grad_optimizer(
      ref.row_pointers[sname], ref.embedding_ids[sname],
      ref.sample_ids[sname], ref.gains[sname], grad, table, slots,
      optimizer=_oracle_name(name), hyperparameters=HYPER[name],
      num_sc_per_device=num_sc, num_scs=num_sc,
      multiply_linear_by_lr=name == "ftrl_by_lr", min_value=lo, max_value=hi)


def _ftrl_pow_bounds(name, table, slots, exp):
  """FTRL's linear slot takes dp = a'^0.5 - a^0.5 times table / lr: one ulp
  of either pow (device and host libraries may round differently) moves it
  by about 2^-24 * a^0.5 * |table| / lr, and the table by that over the
  denominator. Extra absolute error allowed (table, accumulator, linear)."""
  lr, _, _, l2, beta = (float(h) for h in HYPER[name])
  p = np.sqrt(np.maximum(slots[0].astype(np.float64), exp[1]))
  by_lr = name == "ftrl_by_lr"
  lin_err = 4 * 2.0 ** -24 * p * np.abs(table) * (1.0 if by_lr else 1 / lr)
  den = (p + 2 * lr * l2 + beta) if by_lr else (p + beta) / lr + 2 * l2
  return lin_err / den, 0.0, lin_err


@pytest.mark.parametrize("name", sorted(PRIMS))
@pytest.mark.parametrize("kind", ["unique", "hot"])
@pytest.mark.parametrize("num_sc", [1, 4])
def test_optimizer_matches_oracle(name, kind, num_sc):
  rng = np.random.default_rng(zlib.crc32(f"{name}/{kind}/{num_sc}".encode()))
  ids, fs, sname, ref = _case(kind, rng, num_sc)
  spec = fs.table_spec.stacked_table_spec
  shape = (spec.stack_vocab_size, spec.stack_embedding_dim)
  table = rng.normal(0, 0.5, size=shape).astype(np.float32)
  slots = _slots(_oracle_name(name), rng, shape)
  # Hot rows: small-integer gradients, so that every partial sum of a row's
  # gradient is exact and the kernel's summation order cannot matter.
  grad = (rng.normal(size=(ids.shape[0], shape[1])) if kind == "unique" else
          rng.integers(-3, 4, size=(ids.shape[0], shape[1]))).astype(
              np.float32)
  lo, hi = (-0.4, 0.4) if name in ("adam", "f2a") else (None, None)
  out = _bind(name, ref, sname, torch.from_numpy(table).cuda(),
              [torch.from_numpy(s).cuda() for s in slots],
              torch.from_numpy(grad).cuda(), num_sc, min_value=lo,
              max_value=hi)
  exp = _oracle(name, ref, sname, table, slots, grad, num_sc, lo, hi)
  rtol, atol = 1e-5, 1e-6
  extra = _ftrl_pow_bounds(name, table, slots, exp) if name.startswith(
      "ftrl") else (0.0, 0.0, 0.0)
  for g, e, x, what in zip(out, exp, extra, ("table", "slot 0", "slot 1")):
    err = np.abs(g.cpu().numpy().astype(np.float64) - e)
    bound = rtol * np.abs(e) + atol + x
    assert (err <= bound).all(), (
        f"{name} {kind} {what}: max excess {float((err - bound).max())}")
  moved = int((out[0].cpu().numpy() != table).any(axis=1).sum())
  assert moved > 0


@pytest.mark.parametrize("name", ["adam", "ftrl", "f2a"])
def test_optimizer_routes_and_hyperparameter_sources_agree(name):
  """Same bits: CSR read in place vs sorted copy, dense vs per-feature
  gradients, host vs device hyperparameters, and a second identical call."""
  rng = np.random.default_rng(11)
  ids, fs, sname, ref = _case("hot", rng, 1)
  spec = fs.table_spec.stacked_table_spec
  shape = (spec.stack_vocab_size, spec.stack_embedding_dim)
  table = rng.normal(0, 0.5, size=shape).astype(np.float32)
  slots = _slots(name, rng, shape)
  grad = torch.from_numpy(
      rng.normal(size=(ids.shape[0], shape[1])).astype(np.float32)).cuda()

  def run(**kw):
    t = torch.from_numpy(table).cuda()
    s = [torch.from_numpy(x).cuda() for x in slots]
    g = kw.pop("grad", grad)
    out = _bind(name, ref, sname, t, s, g, 1, **kw)
    return [x.cpu().numpy() for x in out]

  base = run(csr_sorted_by_row=False)  # a sorted copy of the entries
  variants = {
      "sorted_by_row": run(csr_sorted_by_row=True),
      "format_order": run(),  # the default reads the CSR in place too
      "device_hyper": run(hyper=[
          torch.tensor(float(h), dtype=torch.float32, device="cuda")
          for h in HYPER[name]]),
      "blocks": run(grad=_device.RowBlocks(
          grad.shape[0], shape[1],
          [(0, grad[:300], shape[1]), (300, grad[300:], shape[1])])),
      "again": run(csr_sorted_by_row=False),
  }
  for what, got in variants.items():
    for g, b in zip(got, base):
      np.testing.assert_array_equal(g, b, err_msg=f"{name} {what}")


@pytest.mark.parametrize("opt_name", ["adam", "adagrad_momentum", "ftrl",
                                      "laprop", "f2a"])
def test_embedding_api_trains_with_every_optimizer(opt_name):
  """Two tables stacked, one feature each, through init_embedding_variables,
  tpu_sparse_dense_matmul and tpu_sparse_dense_matmul_grad (step 3): the
  returned slot variables keep the optimizer's *SlotVariables type and every
  array matches the oracle run with the spec's own hyperparameters."""
  opt = {
      "adam": embedding_spec.AdamOptimizerSpec(learning_rate=0.01),
      "adagrad_momentum": embedding_spec.AdagradMomentumOptimizerSpec(
          learning_rate=0.02, use_nesterov=True),
      "ftrl": embedding_spec.FTRLOptimizerSpec(
          learning_rate=0.05, l1_regularization_strength=0.001,
          multiply_linear_by_learning_rate=True),
      "laprop": embedding_spec.LaPropOptimizerSpec(learning_rate=0.01),
      "f2a": embedding_spec.F2AOptimizerSpec(learning_rate=0.01,
                                             l2_regularization_strength=0.01),
  }[opt_name]
  rng = np.random.default_rng(21)
  batch = 256
  tables = [embedding_spec.TableSpec(
      name=f"t{k}", vocabulary_size=v, embedding_dim=16,
      initializer=embedding_spec.normal(0.1), optimizer=opt, combiner="sum",
      max_ids_per_partition=1 << 16, max_unique_ids_per_partition=1 << 16)
            for k, v in enumerate((500, 900))]
  feats = [embedding_spec.FeatureSpec(
      name=f"f{k}", table_spec=t, input_shape=[batch, 2],
      output_shape=[batch, 16]) for k, t in enumerate(tables)]
  table_stacking.stack_tables(
      feats, ["t0", "t1"], 1, 1,
      stack_to_max_ids_per_partition=lambda n, b: 1 << 16,
      stack_to_max_unique_ids_per_partition=lambda n, b: 1 << 16)
  features = [_zipf(rng, 1.2, t.vocabulary_size, 2 * batch).reshape(batch, 2)
              for t in tables]
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      features, None, feats, 1, 1, num_sc_per_device=1)
  ref = refcpu.preprocess(features, None, feats, 1, 1, num_sc_per_device=1)
  variables = embedding.init_embedding_variables(7, tables,
                                                 num_sparsecore_per_device=1)
  name = next(iter(variables))
  ev = variables[name]
  assert type(ev.slot) is type(opt.slot_variables_initializers())
  table0 = ev.table.cpu().numpy()
  slots0 = [s.cpu().numpy() for s in ev.slot]
  grads = [rng.normal(size=(batch, 16)).astype(np.float32) for _ in feats]
  out = embedding.tpu_sparse_dense_matmul_grad(
      [torch.from_numpy(g).cuda() for g in grads], pre, variables, feats,
      global_device_count=1, num_sc_per_device=1, step=3)
  got = out[name]
  assert type(got.slot) is type(opt.slot_variables_initializers())
  hyper = opt.get_hyperparameters(3)
  exp = refcpu.sparse_dense_matmul_grad_optimizer(
      ref.row_pointers[name], ref.embedding_ids[name], ref.sample_ids[name],
      ref.gains[name], np.concatenate(grads), table0, slots0,
      optimizer=opt_name, hyperparameters=hyper, num_sc_per_device=1,
      num_scs=1, multiply_linear_by_lr=bool(
          getattr(opt, "multiply_linear_by_learning_rate", False)))
  for g, e, what in zip([got.table, *got.slot], exp,
                        ("table", "slot 0", "slot 1")):
    np.testing.assert_allclose(g.cpu().numpy(), e, rtol=1e-4, atol=1e-5,
                               err_msg=f"{opt_name} {what}")
