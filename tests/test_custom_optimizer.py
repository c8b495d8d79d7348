"""Custom optimizer updates on the CPU: lowering, parsing, the register
program, the C-ABI's program checks and the oracle.

The first four tests are the reference's custom_optimizer_lowering_test.py
(lib/nn/tests/custom_optimizer_lowering_test.py:24-118) with numpy in place
of jax.numpy. The rest pin what jax does in the reference and this build
does itself:
  * the register program (`UpdateProgram.compile`) run by a numpy
    interpreter written here must equal the function evaluated directly in
    numpy float32, bit for bit, for functions that keep many values live
    (a register freed too early or an operand swapped fails this);
  * StableHLO in jax's text form (locations, scalar constants broadcast,
    a private function reached by `call`, compare + select) parses to the
    same program as the traced function;
  * the C-ABI refuses malformed programs before touching the device;
  * the oracle's custom update equals its built-in SGD and Adagrad when the
    function is that update, and reproduces the reference's custom-Adagrad
    expectation (tpu_sparse_dense_matmul_grad_test.py:1324-1486).
"""

import ctypes
import pathlib

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core import input_preprocessing
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_optimizer_grad as smog
from jax_tpu_embedding.sparsecore.lib.nn import custom_optimizer_lowering as col
from oracle import refcpu


# --- custom_optimizer_lowering_test.py --------------------------------------

def test_apply_clipping():
  val = np.array([-2.0, 0.0, 2.0, 5.0], np.float32)
  np.testing.assert_allclose(col.apply_clipping(val), val)
  np.testing.assert_allclose(col.apply_clipping(val, min_value=0.0),
                             [0.0, 0.0, 2.0, 5.0])
  np.testing.assert_allclose(col.apply_clipping(val, max_value=3.0),
                             [-2.0, 0.0, 2.0, 3.0])
  np.testing.assert_allclose(
      col.apply_clipping(val, min_value=0.0, max_value=3.0),
      [0.0, 0.0, 2.0, 3.0])


def _sgd(grad, param, lr):
  return param - lr * grad


def test_lower_to_stablehlo_basic():
  text = col.lower_to_stablehlo(_sgd, embedding_dim=4, num_slot_variables=0,
                                num_hyperparameters=1)
  assert isinstance(text, str)
  assert "module" in text
  assert "stablehlo" in text.lower()


def test_lower_to_stablehlo_with_slots_and_clipping():
  def custom_adagrad(grad, param, accum, lr):
    new_accum = accum + grad * grad
    new_param = param - lr * grad / (np.sqrt(new_accum) + 1e-7)
    return new_param, new_accum

  text = col.lower_to_stablehlo(custom_adagrad, embedding_dim=8,
                                num_slot_variables=1, num_hyperparameters=1,
                                min_value=-1.0, max_value=1.0)
  assert isinstance(text, str)
  assert "module" in text
  assert "stablehlo.clamp" in text


def test_wrap_stablehlo_with_limits():
  raw = col.lower_to_stablehlo(_sgd, embedding_dim=4, num_slot_variables=0,
                               num_hyperparameters=1)
  assert col.wrap_stablehlo_with_limits(
      raw, embedding_dim=4, num_slot_variables=0,
      num_hyperparameters=1) == raw
  with_limits = col.wrap_stablehlo_with_limits(
      raw, embedding_dim=4, num_slot_variables=0, num_hyperparameters=1,
      min_value=0.0, max_value=10.0)
  assert isinstance(with_limits, str)
  assert "module" in with_limits
  # The wrapped module clips: evaluated, it holds the table in [0, 10].
  prog = col.parse_stablehlo(with_limits, 0, 1)
  g = np.array([-100.0, 0.0, 1.0, 100.0], np.float32)
  t = np.array([5.0, 5.0, 5.0, 5.0], np.float32)
  (out,) = _run_fields(prog.compile(), [g, t, np.float32(0.1)])
  np.testing.assert_array_equal(
      out, np.array([10.0, 5.0, 5.0 - np.float32(0.1), 0.0], np.float32))


def _thirds(grad, param, lr):
  return param - (lr * np.float32(1.0 / 3.0)) * grad + np.float32(0.1)


@pytest.mark.parametrize("lo,hi", [(-0.123456789, 0.123456789),
                                   (-1e-30, 3.4e38), (None, 2.0 / 3.0)])
def test_printed_constants_keep_their_float32_bits(lo, hi):
  """lower_to_stablehlo -> parse_stablehlo -> compile keeps every constant,
  and the clip bounds, at the float32 bits trace() gives them. Seven
  significant digits would not: 1/3 would come back as 0x3EAAAAAA and
  0.123456789 as 0.1234567985."""
  traced = col.trace(_thirds, 0, 1)
  col._clip_outputs(traced, lo, hi)  # pylint: disable=protected-access
  text = col.lower_to_stablehlo(_thirds, 4, 0, 1, min_value=lo, max_value=hi)
  parsed = col.parse_stablehlo(text, 0, 1)
  want = np.asarray(traced.compile()["imm"], np.float32).view(np.uint32)
  got = np.asarray(parsed.compile()["imm"], np.float32).view(np.uint32)
  np.testing.assert_array_equal(got, want)
  consts = {np.float32(imm).view(np.uint32)
            for name, _, imm in parsed.ops if name == "constant"}
  for v in (1.0 / 3.0, 0.1, lo, hi):
    if v is not None:
      assert np.float32(v).view(np.uint32) in consts, v
  # Evaluated, the parsed module clips at exactly float32(lo) / float32(hi).
  g = np.array([-1e6, 0.0, 1e6], np.float32)
  t = np.zeros(3, np.float32)
  (out,) = _run_fields(parsed.compile(), [g, t, np.float32(1.0)])
  want = _thirds(g, t, np.float32(1.0))
  if hi is not None:
    want = np.minimum(want, np.float32(hi))
  if lo is not None:
    want = np.maximum(want, np.float32(lo))
  np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))
  if hi is not None and hi < 1.0:
    assert out[0] == np.float32(hi)
  if lo is not None and lo > -1.0:
    assert out[2] == np.float32(lo)


# --- the register program ----------------------------------------------------

def _op(code, x, y, z, imm):
  """The kernel's operations (SCEMB_OP_*), restated in numpy float32."""
  f = np.float32
  with np.errstate(all="ignore"):
    return {
        0: lambda: np.full_like(x, imm), 1: lambda: x + y,
        2: lambda: x - y, 3: lambda: x * y, 4: lambda: x / y,
        5: lambda: -x, 6: lambda: np.sqrt(x), 7: lambda: f(1) / np.sqrt(x),
        8: lambda: np.abs(x), 9: lambda: np.exp(x), 10: lambda: np.log(x),
        11: lambda: np.power(x, y), 12: lambda: np.maximum(x, y),
        13: lambda: np.minimum(x, y), 14: lambda: np.sign(x),
        15: lambda: np.tanh(x), 16: lambda: np.log1p(x),
        17: lambda: np.expm1(x), 18: lambda: np.floor(x),
        19: lambda: np.ceil(x), 20: lambda: np.where(x != 0, y, z),
        21: lambda: (x == y).astype(f), 22: lambda: (x != y).astype(f),
        23: lambda: (x < y).astype(f), 24: lambda: (x <= y).astype(f),
        25: lambda: (x > y).astype(f), 26: lambda: (x >= y).astype(f),
        27: lambda: np.minimum(np.maximum(y, x), z),
        28: lambda: ((x != 0) & (y != 0)).astype(f),
        29: lambda: ((x != 0) | (y != 0)).astype(f),
        30: lambda: (x == 0).astype(f),
    }[code]().astype(f)


def _run_fields(fields, inputs):
  """Runs compiled program fields on numpy inputs (gradient, table, slots,
  hyperparameters) as the kernel does: a register file, one op at a time."""
  shape = np.shape(inputs[0])
  regs = [None] * col.MAX_REGISTERS
  for i, v in enumerate(inputs):
    regs[i] = np.broadcast_to(np.asarray(v, np.float32), shape).copy()
  zero = np.zeros(shape, np.float32)
  for k, code in enumerate(fields["op"]):
    a, b, c = (regs[fields[r][k]] for r in ("a", "b", "c"))
    regs[fields["dst"][k]] = _op(code, zero if a is None else a,
                                 zero if b is None else b,
                                 zero if c is None else c,
                                 np.float32(fields["imm"][k]))
  return [regs[r] for r in fields["out"]]


def _ftrl(grad, table, accum, linear, lr, lr_power, l1, l2, beta):
  # sparse_dense_matmul_optimizer_grad_test.py:341-357
  two = np.float32(2.0)
  zero = np.float32(0.0)
  a_new = accum + grad * grad
  p_old = np.power(accum, -lr_power)
  p_new = np.power(a_new, -lr_power)
  delta_p = p_new - p_old
  new_linear = linear + grad - (delta_p / lr) * table
  numerator = np.sign(new_linear) * l1 - new_linear
  denominator = (p_new + beta) / lr + two * l2
  w_new = np.where(np.abs(new_linear) > l1, numerator / denominator, zero)
  return w_new, a_new, new_linear


def _adam(grad, table, m, v, alpha_t, beta_1, beta_2, epsilon_hat):
  # sparse_dense_matmul_optimizer_grad_test.py:475-479
  new_m = beta_1 * m + (1.0 - beta_1) * grad
  new_v = beta_2 * v + (1.0 - beta_2) * (grad * grad)
  return table - alpha_t * new_m / (np.sqrt(new_v) + epsilon_hat), new_m, new_v


def _wide(grad, table, s, h0, h1):
  """Many values live at once: six partial terms combined at the end."""
  terms = [grad * np.float32(k + 1) - s * h1 for k in range(6)]
  total = terms[0]
  for t in terms[1:]:
    total = total + t * t
  return table - total * h0, np.maximum(s, np.abs(grad))


@pytest.mark.parametrize("fn,ns,nh", [
    (_sgd, 0, 1), (_ftrl, 2, 5), (_adam, 2, 4), (_wide, 1, 2)])
def test_compiled_program_equals_numpy(fn, ns, nh):
  rng = np.random.default_rng(7)
  n = 257
  grad = rng.normal(size=n).astype(np.float32)
  table = rng.normal(size=n).astype(np.float32)
  slots = [rng.uniform(0.05, 2.0, size=n).astype(np.float32)
           for _ in range(ns)]
  hyper = [np.float32(x) for x in (0.1, -0.5, 0.001, 0.002, 0.01)[:nh]]
  prog = col.trace(fn, ns, nh)
  fields = prog.compile()
  assert max(fields["dst"]) < col.MAX_REGISTERS
  got = _run_fields(fields, [grad, table, *slots, *hyper])
  want = fn(grad, table, *slots, *hyper)
  want = want if isinstance(want, tuple) else (want,)
  assert len(got) == len(want) == 1 + ns
  for g, w in zip(got, want):
    np.testing.assert_array_equal(g.view(np.int32),
                                  np.asarray(w, np.float32).view(np.int32))
  # Printed and parsed back, the module is the same program.
  again = col.parse_stablehlo(prog.to_stablehlo(8), ns, nh)
  assert again.ops == prog.ops and again.outputs == prog.outputs


# StableHLO as jax writes it for the reference test's update functions with
# (1, 8) operands (jax.jit(fn).lower(...).as_text(dialect="stablehlo")):
# scalar constants broadcast, jnp.clip as a private function, locations.
JAX_ADAGRAD = (pathlib.Path(__file__).parent / "golden" /
               "custom_adagrad_jax.stablehlo").read_text()

JAX_SGD_CLIP = """\
module @jit_sgd_with_clip attributes {mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32} {
  func.func public @main(%arg0: tensor<1x8xf32>, %arg1: tensor<1x8xf32>, %arg2: tensor<1x8xf32>) -> (tensor<1x8xf32> {jax.result_info = "result"}) {
    %cst = stablehlo.constant dense<-2.000000e+00> : tensor<f32>
    %cst_0 = stablehlo.constant dense<5.000000e+00> : tensor<f32>
    %0 = stablehlo.multiply %arg2, %arg0 : tensor<1x8xf32>
    %1 = stablehlo.subtract %arg1, %0 : tensor<1x8xf32>
    %2 = call @clip(%1, %cst, %cst_0) : (tensor<1x8xf32>, tensor<f32>, tensor<f32>) -> tensor<1x8xf32>
    return %2 : tensor<1x8xf32>
  }
  func.func private @clip(%arg0: tensor<1x8xf32>, %arg1: tensor<f32>, %arg2: tensor<f32>) -> tensor<1x8xf32> {
    %0 = stablehlo.broadcast_in_dim %arg1, dims = [] : (tensor<f32>) -> tensor<1x8xf32>
    %1 = stablehlo.maximum %0, %arg0 : tensor<1x8xf32>
    %2 = stablehlo.broadcast_in_dim %arg2, dims = [] : (tensor<f32>) -> tensor<1x8xf32>
    %3 = stablehlo.minimum %2, %1 : tensor<1x8xf32>
    return %3 : tensor<1x8xf32>
  }
}
"""

JAX_WHERE = """\
module @jit_f attributes {mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32} {
  func.func public @main(%arg0: tensor<1x8xf32>, %arg1: tensor<1x8xf32>, %arg2: tensor<1x8xf32>) -> (tensor<1x8xf32> {jax.result_info = "result"}) {
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.broadcast_in_dim %cst, dims = [] : (tensor<f32>) -> tensor<1x8xf32>
    %1 = stablehlo.compare  GT, %arg0, %0,  FLOAT : (tensor<1x8xf32>, tensor<1x8xf32>) -> tensor<1x8xi1>
    %2 = stablehlo.multiply %arg2, %arg0 : tensor<1x8xf32>
    %3 = stablehlo.subtract %arg1, %2 : tensor<1x8xf32>
    %4 = stablehlo.select %1, %3, %arg1 : tensor<1x8xi1>, tensor<1x8xf32>
    return %4 : tensor<1x8xf32>
  }
}
"""


def _adagrad(grad, table, accum, lr):
  new_accum = accum + grad * grad
  return table - lr * grad / np.sqrt(new_accum), new_accum


@pytest.mark.parametrize("text,fn,ns", [
    (JAX_ADAGRAD, _adagrad, 1),
    (JAX_SGD_CLIP, lambda g, t, lr: np.clip(t - lr * g, -2.0, 5.0), 0),
    (JAX_WHERE, lambda g, t, lr: np.where(g > 0, t - lr * g, t), 0),
])
def test_jax_text_parses_to_the_function(text, fn, ns):
  rng = np.random.default_rng(3)
  grad = rng.normal(size=64).astype(np.float32) * 4
  table = rng.normal(size=64).astype(np.float32) * 4
  slots = [rng.uniform(0.1, 1.0, size=64).astype(np.float32)
           for _ in range(ns)]
  lr = np.float32(0.3)
  prog = col.parse_stablehlo(text, ns, 1)
  got = _run_fields(prog.compile(), [grad, table, *slots, lr])
  want = fn(grad, table, *slots, lr)
  want = want if isinstance(want, tuple) else (want,)
  for g, w in zip(got, want):
    np.testing.assert_array_equal(g, np.asarray(w, np.float32))
  # bytes are accepted as the primitive's operand is.
  assert col.parse_stablehlo(text.encode(), ns, 1).ops == prog.ops


def test_parse_rejects_what_the_kernel_cannot_run():
  with pytest.raises(ValueError, match="dot_general"):
    col.parse_stablehlo(JAX_ADAGRAD.replace(
        "stablehlo.sqrt %1", "stablehlo.dot_general %1"), 1, 1)
  with pytest.raises(ValueError, match="@main takes 4 arguments"):
    col.parse_stablehlo(JAX_ADAGRAD, 0, 1)
  with pytest.raises(ValueError, match="per-column constants"):
    col.parse_stablehlo(JAX_WHERE.replace(
        "dense<0.000000e+00> : tensor<f32>",
        "dense<[1.0, 2.0]> : tensor<2xf32>"), 0, 1)
  with pytest.raises(ValueError, match="without a @main"):
    col.parse_stablehlo("module {}", 0, 1)


def test_tracer_errors_and_limits():
  with pytest.raises(TypeError, match="must not branch"):
    col.trace(lambda g, t, lr: t - lr * g if g > 0 else t, 0, 1)
  with pytest.raises(ValueError, match="numpy.sin is not supported"):
    col.trace(lambda g, t, lr: np.sin(t), 0, 1)
  with pytest.raises(ValueError, match="returned 1 values"):
    col.trace(lambda g, t, s, lr: t - lr * g, 1, 1)
  with pytest.raises(ValueError, match="at most 2 slot variables"):
    col.trace(lambda *a: a[1], 3, 1)

  def long(g, t, lr):
    for _ in range(60):
      t = t - lr * g
    return t
  with pytest.raises(ValueError, match="at most 48 are supported"):
    col.trace(long, 0, 1).compile()

  def wide(g, t, lr):
    # 24 values computed before any is combined: with the three inputs, more
    # than the 24 registers (in 47 operations).
    pairs = [(g, t), (t, g), (g, lr), (lr, g), (t, lr), (lr, t)]
    vals = [f(x, y) for x, y in pairs for f in (
        lambda x, y: x + y, lambda x, y: x - y, lambda x, y: x * y,
        lambda x, y: x / y)]
    out = t
    for v in vals:
      out = out + v
    return out
  with pytest.raises(ValueError, match="values live at once"):
    col.trace(wide, 0, 1).compile()


def test_torch_functions_trace():
  torch = pytest.importorskip("torch")

  def fn(g, t, acc, lr):
    new = acc + torch.square(g)
    return t - lr * g * torch.rsqrt(new), new

  prog = col.trace(fn, 1, 1)
  names = [op for op, _, _ in prog.ops]
  assert "rsqrt" in names and names.count("multiply") == 3


# --- the C-ABI's checks ------------------------------------------------------

def _grad_call(program):
  lib = _native.load_library()
  csr = _native.Csr()
  opt = _native.Optimizer()
  opt.kind = _native.OPTIMIZER_CUSTOM
  if program is not None:
    opt.program = ctypes.pointer(program)
  fake = ctypes.c_void_p(256)  # never dereferenced: the checks come first
  return lib.scemb_sparse_dense_matmul_grad_with_optimizer(
      ctypes.byref(csr), fake, 16, fake, 32, 8, ctypes.byref(opt), fake,
      1 << 20, None, None)


def _last_error():
  return _native.load_library().scemb_last_error().decode()


def _fields(prog):
  return prog.compile()


def test_c_abi_refuses_malformed_programs():
  good = _fields(col.trace(_adagrad, 1, 1))
  bad_cases = {
      "without program": None,
      "bad opcode or register": dict(good, op=[99] + good["op"][1:]),
      "reads a register before": dict(good, a=[20] + good["a"][1:]),
      "bad output register": dict(good, out=[23, good["out"][1]]),
  }
  for msg, fields in bad_cases.items():
    prog = None if fields is None else _native.update_program(fields)
    rc = _grad_call(prog)
    assert rc == _native.SCEMB_ERR_INVALID_ARGUMENT, msg
    assert msg in _last_error(), (msg, _last_error())
  too_many = _native.update_program(good)
  too_many.num_ops = 49
  assert _grad_call(too_many) == _native.SCEMB_ERR_INVALID_ARGUMENT
  assert "at most 48 operations" in _last_error()


def test_primitive_program_struct():
  text = col.lower_to_stablehlo(_adagrad, 8, 1, 1)
  s = smog.program_struct(text, 1, 1)
  assert (s.num_slots, s.num_hyperparameters) == (1, 1)
  assert s.num_ops == len(col.parse_stablehlo(text, 1, 1).ops)
  with pytest.raises(ValueError, match="stablehlo must be a string"):
    smog.program_struct(3, 1, 1)
  with pytest.raises(ValueError, match="traced for 1 slot"):
    smog.program_struct(col.trace(_adagrad, 1, 1), 0, 1)


# --- the oracle --------------------------------------------------------------

INPUT_C = np.array([[5], [3], [9], [1], [6], [12], [0], [4], [15], [13],
                    [11], [7], [8], [14], [2], [10]], dtype=np.int32)


def _csr(ids, num_sc, limit=64):
  spec = input_preprocessing.single_feature_spec(
      ids.shape[0], 31, limit, limit, 1, num_sc)
  r = refcpu.preprocess([ids], [np.ones(ids.shape, np.float32)], [spec], 1,
                        1, num_sc_per_device=num_sc)
  n = spec.table_spec.stacked_table_spec.stack_name
  return r.row_pointers[n], r.embedding_ids[n], r.sample_ids[n], r.gains[n]


def test_oracle_custom_adagrad_matches_reference_expectation():
  """tpu_sparse_dense_matmul_grad_test.py:1324-1486 on the oracle: table c
  (32 x 18, rows holding their ids, 4 SparseCores), unit gradients."""
  rp, eid, sid, gains = _csr(INPUT_C, 4, 16)
  table = np.tile(np.arange(32, dtype=np.float32)[:, None], (1, 24))
  sharded = np.asarray(refcpu_shard(table, 4))
  acc = np.zeros_like(sharded)
  new_t, new_a = refcpu.sparse_dense_matmul_grad_custom(
      rp, eid, sid, gains, np.ones((16, 24), np.float32), sharded, [acc],
      update_fn=_adagrad, hyperparameters=[0.01], num_sc_per_device=4,
      num_scs=4)
  expected_t = np.array(
      [-1.000e-02, 3.990e00, 7.990e00, 1.199e01, 1.600e01, 2.000e01,
       2.400e01, 2.800e01, 9.900e-01, 4.990e00, 8.990e00, 1.299e01, 1.700e01,
       2.100e01, 2.500e01, 2.900e01, 1.990e00, 5.990e00, 9.990e00, 1.399e01,
       1.800e01, 2.200e01, 2.600e01, 3.000e01, 2.990e00, 6.990e00, 1.099e01,
       1.499e01, 1.900e01, 2.300e01, 2.700e01, 3.100e01], np.float32)
  expected_a = np.array(([1.0] * 4 + [0.0] * 4) * 4, np.float32)
  np.testing.assert_allclose(new_t[:, :18], np.tile(expected_t[:, None],
                                                    (1, 18)))
  np.testing.assert_allclose(new_a[:, :18], np.tile(expected_a[:, None],
                                                    (1, 18)))


def refcpu_shard(table, num_sc):
  v = table.shape[0]
  out = np.empty_like(table)
  for r in range(v):
    out[(r % num_sc) * (v // num_sc) + r // num_sc] = table[r]
  return out


def test_oracle_custom_equals_builtin_updates():
  """Multi-hot ids with weights: the custom path of the oracle (its C SGD's
  gradient sums, then the function in numpy) equals its built-in SGD and
  Adagrad bit for bit when the function is that update."""
  rng = np.random.default_rng(11)
  ids = rng.integers(0, 32, size=(64, 6)).astype(np.int32)
  spec = input_preprocessing.single_feature_spec(64, 31, 256, 256, 1, 4)
  w = rng.uniform(0.5, 1.5, size=ids.shape).astype(np.float32)
  r = refcpu.preprocess([ids], [w], [spec], 1, 1, num_sc_per_device=4)
  n = spec.table_spec.stacked_table_spec.stack_name
  args = (r.row_pointers[n], r.embedding_ids[n], r.sample_ids[n], r.gains[n])
  grad = rng.normal(size=(64, 8)).astype(np.float32)
  table = rng.normal(size=(32, 8)).astype(np.float32)
  acc = rng.uniform(0.1, 1.0, size=(32, 8)).astype(np.float32)
  common = dict(num_sc_per_device=4, num_scs=4)

  (custom,) = refcpu.sparse_dense_matmul_grad_custom(
      *args, grad, table, [], update_fn=_sgd, hyperparameters=[0.05],
      **common)
  builtin = refcpu.sparse_dense_matmul_grad(*args, grad, table.copy(),
                                            learning_rate=0.05, **common)
  np.testing.assert_array_equal(custom, builtin)

  custom_t, custom_a = refcpu.sparse_dense_matmul_grad_custom(
      *args, grad, table, [acc], update_fn=_adagrad,
      hyperparameters=[0.05], **common)
  bt, ba = refcpu.sparse_dense_matmul_grad(*args, grad, table, acc,
                                           learning_rate=0.05, **common)
  np.testing.assert_array_equal(custom_t, bt)
  np.testing.assert_array_equal(custom_a, ba)
