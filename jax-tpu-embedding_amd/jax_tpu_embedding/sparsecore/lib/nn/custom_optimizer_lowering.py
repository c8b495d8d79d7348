"""Custom optimizer updates as element-wise programs (reference:
lib/nn/custom_optimizer_lowering.py).

The reference traces a CustomOptimizerSpec's function of
(gradient, table, *slots, *hyperparameters) with jax into StableHLO text
(`lower_to_stablehlo`, :79-123), optionally wrapped with the clipping of the
table (`wrap_stablehlo_with_limits`, :126-163), and the SparseCore compiler
runs that module on every touched embedding row. jax is not part of this
build, so the same pieces are built here on an element-wise program:

  trace(fn, ...)         calls `fn` on tracer values that record every
                         operation; `fn` may use Python arithmetic, numpy
                         (ufuncs, np.where, np.clip, ...) or torch functions
                         on its arguments, and constants;
  parse_stablehlo(text)  reads the element-wise subset of StableHLO that such
                         functions lower to (jax's text form: func.func
                         @main, private helper functions reached by
                         func.call, stablehlo.* element-wise ops, scalar or
                         splat constants, broadcast_in_dim / reshape /
                         convert of them);
  UpdateProgram          the result: straight-line operations over values,
                         printable as StableHLO (`to_stablehlo`) and
                         compiled to the kernel's register program
                         (`compile`, scemb_update_program_t).

`lower_to_stablehlo` and `wrap_stablehlo_with_limits` keep the reference's
names and arguments and return StableHLO text, so specs and primitive
operands written for the reference carry over.
"""

from __future__ import annotations

import math
import re
from typing import Any, Callable, Sequence

import numpy as np

# Operations (StableHLO names), their opcode in scemb_update_program_t
# (SCEMB_OP_* of include/scemb.h, same order) and arity.
_OPS = {
    "constant": (0, 0), "add": (1, 2), "subtract": (2, 2),
    "multiply": (3, 2), "divide": (4, 2), "negate": (5, 1), "sqrt": (6, 1),
    "rsqrt": (7, 1), "abs": (8, 1), "exponential": (9, 1), "log": (10, 1),
    "power": (11, 2), "maximum": (12, 2), "minimum": (13, 2),
    "sign": (14, 1), "tanh": (15, 1), "log_plus_one": (16, 1),
    "exponential_minus_one": (17, 1), "floor": (18, 1), "ceil": (19, 1),
    "select": (20, 3), "compare_EQ": (21, 2), "compare_NE": (22, 2),
    "compare_LT": (23, 2), "compare_LE": (24, 2), "compare_GT": (25, 2),
    "compare_GE": (26, 2), "clamp": (27, 3), "and": (28, 2), "or": (29, 2),
    "not": (30, 1),
}
_BOOL_OPS = {"compare_EQ", "compare_NE", "compare_LT", "compare_LE",
             "compare_GT", "compare_GE", "and", "or", "not"}

MAX_OPS = 48          # SCEMB_PROGRAM_MAX_OPS
MAX_REGISTERS = 24    # SCEMB_PROGRAM_MAX_REGISTERS
MAX_SLOTS = 2
MAX_HYPERPARAMETERS = 8


class UpdateProgram:
  """Straight-line element-wise update.

  Values 0.. are the inputs (gradient, table, the slot variables, the
  hyperparameters); operation i defines value num_inputs + i as
  `(name, args, imm)` (imm: the constant of a "constant"); `outputs` are the
  values of the new table and the new slot variables.
  """

  def __init__(self, num_slots: int, num_hyperparameters: int):
    self.num_slots = num_slots
    self.num_hyperparameters = num_hyperparameters
    self.ops: list[tuple[str, tuple[int, ...], float | None]] = []
    self.outputs: list[int] = []
    self._consts: dict[int, int] = {}

  @property
  def num_inputs(self) -> int:
    return 2 + self.num_slots + self.num_hyperparameters

  def emit(self, name: str, args: Sequence[int] = (),
           imm: float | None = None) -> int:
    if name not in _OPS:
      raise ValueError(f"custom optimizer: unsupported operation {name}")
    if name == "constant":
      bits = int(np.float32(imm).view(np.uint32))
      if bits in self._consts:
        return self._consts[bits]
    self.ops.append((name, tuple(args), None if imm is None else
                     float(np.float32(imm))))
    vid = self.num_inputs + len(self.ops) - 1
    if name == "constant":
      self._consts[bits] = vid
    return vid

  # -- StableHLO -----------------------------------------------------------

  def to_stablehlo(self, embedding_dim: int = 1) -> str:
    """The program as a StableHLO module in jax's text form: every value a
    tensor<1 x embedding_dim> (booleans of i1)."""
    ty = f"tensor<1x{int(embedding_dim)}xf32>"
    bty = f"tensor<1x{int(embedding_dim)}xi1>"
    names = [f"%arg{i}" for i in range(self.num_inputs)]
    lines = []
    for i, (name, args, imm) in enumerate(self.ops):
      vid = self.num_inputs + i
      out = f"%{i}"
      names.append(out)
      a = [names[x] for x in args]
      if name == "constant":
        lines.append(f"    {out} = stablehlo.constant dense<{_fmt(imm)}> : "
                     f"{ty}")
      elif name.startswith("compare_"):
        lines.append(f"    {out} = stablehlo.compare  {name[8:]}, {a[0]}, "
                     f"{a[1]},  FLOAT : ({ty}, {ty}) -> {bty}")
      elif name == "select":
        lines.append(f"    {out} = stablehlo.select {a[0]}, {a[1]}, {a[2]} "
                     f": {bty}, {ty}")
      elif name in ("and", "or", "not"):
        lines.append(f"    {out} = stablehlo.{name} {', '.join(a)} : {bty}")
      else:
        lines.append(f"    {out} = stablehlo.{name} {', '.join(a)} : {ty}")
      del vid
    args = ", ".join(f"%arg{i}: {ty}" for i in range(self.num_inputs))
    results = ", ".join(
        f'{ty} {{jax.result_info = "result[{k}]"}}'
        for k in range(len(self.outputs)))
    ret = ", ".join(names[v] for v in self.outputs)
    rtys = ", ".join(ty for _ in self.outputs)
    return ("module @jit_custom_optimizer attributes {mhlo.num_partitions = "
            "1 : i32, mhlo.num_replicas = 1 : i32} {\n"
            f"  func.func public @main({args}) -> ({results}) {{\n" +
            "".join(line + "\n" for line in lines) +
            f"    return {ret} : {rtys}\n  }}\n}}\n")

  # -- the kernel's register program ----------------------------------------

  def compile(self) -> dict:
    """Register allocation: inputs in registers 0.. (gradient, table, slots,
    hyperparameters), each operation into a register freed by values whose
    last use is behind it. Returns the fields of scemb_update_program_t."""
    if len(self.ops) > MAX_OPS:
      raise ValueError(f"custom optimizer: {len(self.ops)} operations, at "
                       f"most {MAX_OPS} are supported")
    n_in = self.num_inputs
    last_use = {}
    for i, (_, args, _) in enumerate(self.ops):
      for a in args:
        last_use[a] = i
    keep = set(self.outputs)
    reg = {v: v for v in range(n_in)}
    free = [r for r in range(MAX_REGISTERS - 1, n_in - 1, -1)]
    fields = {k: [] for k in ("op", "dst", "a", "b", "c", "imm")}
    for i, (name, args, imm) in enumerate(self.ops):
      srcs = [reg[a] for a in args] + [0] * (3 - len(args))
      # Values used for the last time here give their registers back first,
      # so the result may reuse one.
      for a in set(args):
        if last_use.get(a) == i and a not in keep:
          free.append(reg[a])
      if not free:
        raise ValueError("custom optimizer: more than "
                         f"{MAX_REGISTERS} values live at once")
      dst = free.pop()
      reg[n_in + i] = dst
      code, _ = _OPS[name]
      fields["op"].append(code)
      fields["dst"].append(dst)
      fields["a"].append(srcs[0])
      fields["b"].append(srcs[1])
      fields["c"].append(srcs[2])
      fields["imm"].append(0.0 if imm is None else imm)
      if n_in + i not in last_use and n_in + i not in keep:
        free.append(dst)
    fields["out"] = [reg[v] for v in self.outputs]
    fields["num_slots"] = self.num_slots
    fields["num_hyperparameters"] = self.num_hyperparameters
    return fields


def _fmt(x: float) -> str:
  """The float32 value of x in decimal with 9 significant digits, which is
  enough for the text to parse back to the same float32 bits."""
  if math.isnan(x):
    return "0x7FC00000"
  if math.isinf(x):
    return "0x7F800000" if x > 0 else "0xFF800000"
  f = float(np.float32(x))
  if math.isinf(f):  # a finite double beyond float32's range
    return "0x7F800000" if f > 0 else "0xFF800000"
  return f"{f:.8e}" if f != 0 or math.copysign(1, f) > 0 else "-0.00000000e+00"


# ---------------------------------------------------------------------------
# Tracing.
# ---------------------------------------------------------------------------

_UFUNCS = {
    np.add: "add", np.subtract: "subtract", np.multiply: "multiply",
    np.divide: "divide", np.true_divide: "divide", np.negative: "negate",
    np.positive: None, np.sqrt: "sqrt", np.absolute: "abs",
    np.exp: "exponential", np.log: "log", np.power: "power",
    np.float_power: "power", np.maximum: "maximum", np.minimum: "minimum",
    np.fmax: "maximum", np.fmin: "minimum", np.sign: "sign", np.tanh: "tanh",
    np.log1p: "log_plus_one", np.expm1: "exponential_minus_one",
    np.floor: "floor", np.ceil: "ceil", np.square: "square",
    np.reciprocal: "reciprocal", np.equal: "compare_EQ",
    np.not_equal: "compare_NE", np.less: "compare_LT",
    np.less_equal: "compare_LE", np.greater: "compare_GT",
    np.greater_equal: "compare_GE", np.logical_and: "and",
    np.logical_or: "or", np.logical_not: "not",
}


class Traced:
  """A value of a traced update: arithmetic on it is recorded."""

  __array_priority__ = 1000

  def __init__(self, prog: UpdateProgram, vid: int, is_bool: bool = False):
    self._prog = prog
    self._vid = vid
    self._bool = is_bool

  # Python operators.
  def __add__(self, o): return _apply("add", self, o)
  def __radd__(self, o): return _apply("add", o, self)
  def __sub__(self, o): return _apply("subtract", self, o)
  def __rsub__(self, o): return _apply("subtract", o, self)
  def __mul__(self, o): return _apply("multiply", self, o)
  def __rmul__(self, o): return _apply("multiply", o, self)
  def __truediv__(self, o): return _apply("divide", self, o)
  def __rtruediv__(self, o): return _apply("divide", o, self)
  def __pow__(self, o): return _apply("power", self, o)
  def __rpow__(self, o): return _apply("power", o, self)
  def __neg__(self): return _apply("negate", self)
  def __pos__(self): return self
  def __abs__(self): return _apply("abs", self)
  def __lt__(self, o): return _apply("compare_LT", self, o)
  def __le__(self, o): return _apply("compare_LE", self, o)
  def __gt__(self, o): return _apply("compare_GT", self, o)
  def __ge__(self, o): return _apply("compare_GE", self, o)
  def __eq__(self, o): return _apply("compare_EQ", self, o)  # type: ignore[override]
  def __ne__(self, o): return _apply("compare_NE", self, o)  # type: ignore[override]
  def __and__(self, o): return _apply("and", self, o)
  def __or__(self, o): return _apply("or", self, o)
  def __invert__(self): return _apply("not", self)
  __hash__ = None  # type: ignore[assignment]

  def __bool__(self):
    raise TypeError(
        "custom optimizer functions must not branch on traced values; "
        "use np.where / np.maximum / np.clip instead")

  def __float__(self):
    raise TypeError("a traced value has no concrete float value")

  # numpy.
  def __array_ufunc__(self, ufunc, method, *inputs, **kwargs):
    if method != "__call__" or kwargs.get("out") is not None:
      return NotImplemented
    name = _UFUNCS.get(ufunc, "unsupported")
    if name == "unsupported":
      raise ValueError(f"custom optimizer: numpy.{ufunc.__name__} is not "
                       "supported")
    if name is None:
      return inputs[0]
    return _apply(name, *inputs)

  def __array_function__(self, func, types, args, kwargs):
    if func is np.where:
      return _apply("select", *args)
    if func is np.clip:
      x, lo, hi = args[0], args[1], args[2]
      return apply_clipping(x, lo, hi)
    if func in (np.asarray, np.array):
      return args[0]
    raise ValueError(f"custom optimizer: numpy.{func.__name__} is not "
                     "supported")

  # torch.
  @classmethod
  def __torch_function__(cls, func, types, args=(), kwargs=None):
    kwargs = kwargs or {}
    name = getattr(func, "__name__", "")
    table = {
        "add": "add", "sub": "subtract", "subtract": "subtract",
        "mul": "multiply", "multiply": "multiply", "div": "divide",
        "true_divide": "divide", "neg": "negate", "negative": "negate",
        "sqrt": "sqrt", "rsqrt": "rsqrt", "abs": "abs", "exp": "exponential",
        "log": "log", "pow": "power", "maximum": "maximum",
        "minimum": "minimum", "sign": "sign", "tanh": "tanh",
        "log1p": "log_plus_one", "expm1": "exponential_minus_one",
        "floor": "floor", "ceil": "ceil", "square": "square",
        "reciprocal": "reciprocal", "where": "select", "eq": "compare_EQ",
        "ne": "compare_NE", "lt": "compare_LT", "le": "compare_LE",
        "gt": "compare_GT", "ge": "compare_GE", "logical_and": "and",
        "logical_or": "or", "logical_not": "not",
    }
    if name in ("clamp", "clip"):
      lo = kwargs.get("min", args[1] if len(args) > 1 else None)
      hi = kwargs.get("max", args[2] if len(args) > 2 else None)
      return apply_clipping(args[0], lo, hi)
    if name not in table:
      raise ValueError(f"custom optimizer: torch.{name} is not supported")
    return _apply(table[name], *args)


def _value(prog: UpdateProgram, x) -> Traced:
  if isinstance(x, Traced):
    return x
  if hasattr(x, "item") and getattr(x, "ndim", 0) == 0:
    x = x.item()
  if isinstance(x, (bool, int, float, np.bool_, np.integer, np.floating)):
    return Traced(prog, prog.emit("constant", (), float(x)))
  raise ValueError("custom optimizer: operands must be traced values or "
                   f"scalar constants, got {type(x).__name__}")


def _apply(name: str, *operands) -> Traced:
  prog = next(o._prog for o in operands if isinstance(o, Traced))
  vals = [_value(prog, o) for o in operands]
  ids = [v._vid for v in vals]
  if name == "square":
    return Traced(prog, prog.emit("multiply", (ids[0], ids[0])))
  if name == "reciprocal":
    one = prog.emit("constant", (), 1.0)
    return Traced(prog, prog.emit("divide", (one, ids[0])))
  if name == "select":
    # np.where(cond, a, b): a numeric condition means cond != 0.
    return Traced(prog, prog.emit("select", ids))
  return Traced(prog, prog.emit(name, ids), name in _BOOL_OPS)


def apply_clipping(val, min_value=None, max_value=None):
  """Clips the table values to [min_value, max_value] (either may be None),
  for traced values and numpy arrays alike (:62-76 of the reference)."""
  if isinstance(val, Traced):
    if min_value is not None and max_value is not None:
      return _apply("clamp", min_value, val, max_value)
    if min_value is not None:
      return _apply("maximum", val, min_value)
    if max_value is not None:
      return _apply("minimum", val, max_value)
    return val
  val = np.asarray(val)
  if min_value is not None:
    val = np.maximum(val, np.float32(min_value))
  if max_value is not None:
    val = np.minimum(val, np.float32(max_value))
  return val


def trace(custom_computation_fn: Callable[..., Any],
          num_slot_variables: int = 0,
          num_hyperparameters: int = 1) -> UpdateProgram:
  """The program of `fn(gradient, table, *slots, *hyperparameters)`, which
  returns the new table or (new table, *new slots)."""
  if not 0 <= num_slot_variables <= MAX_SLOTS:
    raise ValueError(f"custom optimizer: at most {MAX_SLOTS} slot variables "
                     "are supported")
  if not 0 <= num_hyperparameters <= MAX_HYPERPARAMETERS:
    raise ValueError(f"custom optimizer: at most {MAX_HYPERPARAMETERS} "
                     "hyperparameters are supported")
  prog = UpdateProgram(num_slot_variables, num_hyperparameters)
  args = [Traced(prog, i) for i in range(prog.num_inputs)]
  out = custom_computation_fn(*args)
  outs = list(out) if isinstance(out, (list, tuple)) else [out]
  if len(outs) != 1 + num_slot_variables:
    raise ValueError(
        f"custom optimizer returned {len(outs)} values; expected the table "
        f"and {num_slot_variables} slot variables")
  prog.outputs = [_value(prog, o)._vid for o in outs]
  return prog


# ---------------------------------------------------------------------------
# StableHLO text.
# ---------------------------------------------------------------------------

_FUNC_RE = re.compile(
    r"func\.func\s+(?:public\s+|private\s+)?@([\w$.\-]+)\s*\((.*?)\)\s*"
    r"(?:->\s*(.*?))?\s*(?:attributes\s*\{.*?\}\s*)?\{\s*$")
_ASSIGN_RE = re.compile(r"^(%[\w#:]+(?:\s*,\s*%[\w#:]+)*)\s*=\s*(.*)$")
_CONST_RE = re.compile(r"dense<\s*([^>]*?)\s*>")


def _parse_float(tok: str) -> float:
  tok = tok.strip()
  if tok in ("true", "false"):
    return 1.0 if tok == "true" else 0.0
  if tok.lower().startswith("0x"):
    bits = int(tok, 16)
    return float(np.uint32(bits).view(np.float32))
  return float(tok)


def _split_operands(text: str) -> list[str]:
  return [t.strip() for t in text.split(",") if t.strip()]


def _parse_functions(text: str) -> dict:
  funcs: dict[str, dict] = {}
  cur = None
  for raw in text.splitlines():
    line = raw.strip()
    if not line or line.startswith("//"):
      continue
    m = _FUNC_RE.search(line)
    if m:
      params = re.findall(r"(%[\w#]+)\s*:", m.group(2))
      cur = {"params": params, "body": []}
      funcs[m.group(1)] = cur
      continue
    if cur is None:
      continue
    if line.startswith("}"):
      cur = None
      continue
    cur["body"].append(line)
  if "main" not in funcs:
    raise ValueError("StableHLO module without a @main function")
  return funcs


def _inline(funcs: dict, name: str, args: list, prog: UpdateProgram,
            depth: int = 0) -> list:
  """Emits the body of function `name` with its parameters bound to `args`
  (program values); returns the program values it returns."""
  if depth > 16:
    raise ValueError("StableHLO calls nested too deeply")
  f = funcs[name]
  if len(args) != len(f["params"]):
    raise ValueError(f"call of @{name} with {len(args)} arguments")
  env = dict(zip(f["params"], args))

  def get(tok):
    tok = tok.strip()
    if tok not in env:
      raise ValueError(f"StableHLO value {tok} used before it is defined")
    return env[tok]

  for line in f["body"]:
    body = line.split(" loc(")[0].strip()
    if body.startswith("return") or body.startswith("func.return") or (
        body.startswith("stablehlo.return")):
      ops = body.split(None, 1)[1] if " " in body else ""
      ops = ops.split(":")[0]
      return [get(t) for t in _split_operands(ops)]
    m = _ASSIGN_RE.match(body)
    if not m:
      raise ValueError(f"unsupported StableHLO line: {line}")
    lhs = [t.strip() for t in m.group(1).split(",")]
    rhs = m.group(2)
    opm = re.match(r"\"?([\w.]+)\"?\s*(.*)$", rhs)
    if not opm:
      raise ValueError(f"unsupported StableHLO line: {line}")
    opname, rest = opm.group(1), opm.group(2)
    if opname in ("func.call", "call"):
      cm = re.match(r"@([\w$.\-]+)\s*\(([^)]*)\)", rest)
      if not cm:
        raise ValueError(f"unsupported call: {line}")
      outs = _inline(funcs, cm.group(1),
                     [get(t) for t in _split_operands(cm.group(2))], prog,
                     depth + 1)
      if len(lhs) == 1 and ":" in lhs[0]:
        base = lhs[0].split(":")[0]
        for k, v in enumerate(outs):
          env[f"{base}#{k}"] = v
        env[base] = outs[0]
      else:
        for k, t in enumerate(lhs):
          env[t] = outs[k]
      continue
    if not opname.startswith("stablehlo."):
      raise ValueError(f"unsupported StableHLO operation {opname}")
    op = opname[len("stablehlo."):]
    target = lhs[0]
    if op == "constant":
      cm = _CONST_RE.search(rest)
      if not cm:
        raise ValueError(f"unsupported constant: {line}")
      val = cm.group(1)
      if val.startswith("["):
        vals = {v.strip() for v in val.strip("[]").split(",")}
        if len(vals) != 1:
          raise ValueError("custom optimizer: per-column constants are not "
                           "supported")
        val = vals.pop()
      env[target] = prog.emit("constant", (), _parse_float(val))
      continue
    operand_text = rest.split(":")[0]
    if op in ("broadcast_in_dim", "reshape", "convert",
              "optimization_barrier"):
      first = re.findall(r"%[\w#]+", operand_text)[0]
      env[target] = get(first)
      continue
    if op == "compare":
      cm = re.match(r"\s*(\w+)\s*,\s*(%[\w#]+)\s*,\s*(%[\w#]+)", rest)
      if not cm:
        raise ValueError(f"unsupported compare: {line}")
      env[target] = prog.emit(f"compare_{cm.group(1)}",
                              (get(cm.group(2)), get(cm.group(3))))
      continue
    names = {"power": "power", "add": "add", "subtract": "subtract",
             "multiply": "multiply", "divide": "divide", "negate": "negate",
             "sqrt": "sqrt", "rsqrt": "rsqrt", "abs": "abs",
             "exponential": "exponential", "log": "log",
             "maximum": "maximum", "minimum": "minimum", "sign": "sign",
             "tanh": "tanh", "log_plus_one": "log_plus_one",
             "exponential_minus_one": "exponential_minus_one",
             "floor": "floor", "ceil": "ceil", "select": "select",
             "clamp": "clamp", "and": "and", "or": "or", "not": "not"}
    if op not in names:
      raise ValueError(f"custom optimizer: StableHLO operation {op} is not "
                       "supported")
    args_ = [get(t) for t in re.findall(r"%[\w#]+", operand_text)]
    if len(args_) != _OPS[names[op]][1]:
      raise ValueError(f"unexpected operand count in: {line}")
    env[target] = prog.emit(names[op], args_)
  raise ValueError(f"function @{name} has no return")


def parse_stablehlo(stablehlo: str | bytes, num_slot_variables: int,
                    num_hyperparameters: int) -> UpdateProgram:
  """The program of a StableHLO update module (the reference primitive's
  `stablehlo` operand)."""
  text = stablehlo.decode("utf-8") if isinstance(stablehlo, bytes) else str(
      stablehlo)
  funcs = _parse_functions(text)
  prog = UpdateProgram(num_slot_variables, num_hyperparameters)
  if len(funcs["main"]["params"]) != prog.num_inputs:
    raise ValueError(
        f"StableHLO @main takes {len(funcs['main']['params'])} arguments; "
        f"expected gradient, table, {num_slot_variables} slot variables and "
        f"{num_hyperparameters} hyperparameters")
  outs = _inline(funcs, "main", list(range(prog.num_inputs)), prog)
  if len(outs) != 1 + num_slot_variables:
    raise ValueError(f"StableHLO @main returns {len(outs)} values; expected "
                     f"{1 + num_slot_variables}")
  prog.outputs = outs
  return prog


def lower_to_stablehlo(custom_computation_fn: Callable[..., Any],
                       embedding_dim: int = 1, num_slot_variables: int = 0,
                       num_hyperparameters: int = 1,
                       min_value: float | None = None,
                       max_value: float | None = None) -> str:
  """StableHLO text of the traced update, with the table clipped to
  [min_value, max_value] when given (:79-123 of the reference)."""
  prog = trace(custom_computation_fn, num_slot_variables, num_hyperparameters)
  _clip_outputs(prog, min_value, max_value)
  return prog.to_stablehlo(embedding_dim)


def wrap_stablehlo_with_limits(stablehlo: str | bytes, embedding_dim: int,
                               num_slot_variables: int,
                               num_hyperparameters: int,
                               min_value: float | None = None,
                               max_value: float | None = None) -> str:
  """The module with the table output clipped; unchanged without limits
  (:126-163 of the reference)."""
  text = stablehlo.decode("utf-8") if isinstance(stablehlo, bytes) else str(
      stablehlo)
  if min_value is None and max_value is None:
    return text
  prog = parse_stablehlo(text, num_slot_variables, num_hyperparameters)
  _clip_outputs(prog, min_value, max_value)
  return prog.to_stablehlo(embedding_dim)


def _clip_outputs(prog: UpdateProgram, min_value, max_value) -> None:
  if min_value is None and max_value is None:
    return
  table = Traced(prog, prog.outputs[0])
  prog.outputs[0] = _value(prog, apply_clipping(table, min_value,
                                                max_value))._vid
