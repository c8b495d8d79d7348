"""Table / feature / stack specs (reference: lib/nn/embedding_spec.py).

The dataclasses keep the reference's field names, defaults and stacking
rules (``FeatureIdTransformation`` :918-938, ``TableSettingInStack``
:940-977, ``TableSpec`` :979-1118, ``FeatureSpec`` :1120-1166,
``StackedTableSpec`` :1169-1205, ``QuantizationConfig`` :1207-1223) so feature
specs written for the reference work unchanged. Optimizers in scope are SGD
(:377-412) and Adagrad (:415-460); learning rates may be numbers, 0-d torch
tensors or callables of the step.

Initializers are callables ``init(generator, shape)`` returning a float32
array; ``init_embedding_variables`` calls them with a ``torch.Generator`` on
the GPU. ``constant``, ``zeros`` and ``normal`` below cover the reference
defaults.
"""

from __future__ import annotations

import dataclasses
import inspect
from typing import Any, Callable, NamedTuple, Sequence

from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd

DEFAULT_ACTIVATION_MEM_BYTES_LIMIT: int = 2048 * 1024

CallableTableInitializer = Callable[..., Any]
LearningRate = Any


# ---------------------------------------------------------------------------
# Initializers.
# ---------------------------------------------------------------------------


def _torch():
  import torch  # pylint: disable=g-import-not-at-top

  return torch


def constant(value: float) -> CallableTableInitializer:
  """Fills the table with `value` (jax.nn.initializers.constant)."""

  def init(generator, shape, device=None):
    del generator
    t = _torch()
    return t.full(tuple(shape), float(value), dtype=t.float32, device=device)

  init.constant_value = float(value)
  return init


def zeros(generator=None, shape=(), device=None):
  t = _torch()
  del generator
  return t.zeros(tuple(shape), dtype=t.float32, device=device)


def normal(stddev: float = 0.01) -> CallableTableInitializer:
  """N(0, stddev^2) entries (jax.nn.initializers.normal)."""

  def init(generator, shape, device=None):
    t = _torch()
    out = t.empty(tuple(shape), dtype=t.float32, device=device)
    out.normal_(0.0, float(stddev), generator=generator)
    return out

  return init


# ---------------------------------------------------------------------------
# Optimizers.
# ---------------------------------------------------------------------------


class SGDSlotVariables(NamedTuple):
  pass


class AdagradSlotVariables(NamedTuple):
  accumulator: Any


class OptimizerSpec:
  """Base of the optimizer specs (embedding_spec.py:122-247)."""

  _float_params: tuple[str, ...] = ()
  _bool_params: tuple[str, ...] = ()

  def __init__(self, learning_rate: LearningRate):
    self.learning_rate = learning_rate

  def get_learning_rate(self, step=None):
    """The learning rate: a float, a 0-d tensor, or learning_rate(step)."""
    lr = self.learning_rate
    if callable(lr):
      args = inspect.getfullargspec(lr).args
      num_args = len(args) if inspect.isfunction(lr) else len(args) - 1
      if num_args == 0:
        return lr()
      if num_args == 1:
        if step is None:
          raise ValueError(
              f"Specified learning rate callable {lr} requires a `step` "
              "argument to be specified.")
        return lr(step)
      raise ValueError(
          "Learning rate callbacks should either take no parameters, or a "
          "single step count argument.")
    return lr

  def get_hyperparameters(self, step=None) -> tuple:
    return (self.get_learning_rate(step),)

  def slot_variables_initializers(self) -> tuple:
    return ()

  def slot_variables_count(self) -> int:
    return len(self.slot_variables_initializers())

  def get_optimizer_primitive(self):
    raise NotImplementedError

  def short_name(self) -> str:
    raise NotImplementedError

  def __hash__(self) -> int:
    raise NotImplementedError

  def __eq__(self, other: object) -> bool:
    if not isinstance(other, OptimizerSpec):
      return False
    return self.__hash__() == other.__hash__()

  def get_float_params(self) -> dict[str, float]:
    return {p: float(getattr(self, p)) for p in self._float_params
            if hasattr(self, p)}

  def get_bool_params(self) -> dict[str, bool]:
    return {p: bool(getattr(self, p)) for p in self._bool_params
            if hasattr(self, p)}


class SGDOptimizerSpec(OptimizerSpec):
  """Stochastic gradient descent: table -= lr * grad."""

  def __init__(self, learning_rate: LearningRate = 0.001):
    super().__init__(learning_rate=learning_rate)

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate),))

  def short_name(self) -> str:
    return "sgd"

  def slot_variables_initializers(self) -> tuple:
    return SGDSlotVariables()

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_grad_with_sgd
            .tpu_sparse_dense_matmul_grad_with_sgd_primitive)


class AdagradOptimizerSpec(OptimizerSpec):
  """Adagrad with an accumulator slot initialised to a constant."""

  _float_params = ("initial_accumulator_value",)

  def __init__(self, learning_rate: LearningRate = 0.001,
               initial_accumulator_value: float = 0.1):
    super().__init__(learning_rate=learning_rate)
    self.initial_accumulator_value = initial_accumulator_value

  def slot_variables_initializers(self) -> tuple:
    return AdagradSlotVariables(
        accumulator=constant(self.initial_accumulator_value))

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate),
                 _hashable(self.initial_accumulator_value)))

  def short_name(self) -> str:
    return "adagrad"

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_grad_with_adagrad
            .tpu_sparse_dense_matmul_grad_with_adagrad_primitive)


def _hashable(v):
  try:
    hash(v)
    return v
  except TypeError:
    return id(v)


# ---------------------------------------------------------------------------
# Specs.
# ---------------------------------------------------------------------------


@dataclasses.dataclass(eq=True, frozen=True)
class FeatureIdTransformation:
  """Row/column transformation of a feature's ids inside its stack."""

  row_offset: int = 0
  col_offset: int = 0
  col_shift: int = 0


@dataclasses.dataclass(eq=True, frozen=True, kw_only=True)
class TableSettingInStack:
  """Placement of a table inside its stacked table."""

  stack_name: str
  padded_vocab_size: int
  padded_embedding_dim: int
  row_offset_in_shard: int = 0
  shard_rotation: int = 0


@dataclasses.dataclass(frozen=True, slots=True, kw_only=True)
class QuantizationConfig:
  """Per-table quantization parameters (None means disabled)."""

  min_value: float
  max_value: float
  num_buckets: int

  def __post_init__(self):
    if self.num_buckets < 2:
      raise ValueError("num_buckets must be ≥ 2.")
    if self.min_value >= self.max_value:
      raise ValueError("min_value must be < max_value.")

  def as_tuple(self) -> tuple[float, float, int]:
    return (self.min_value, self.max_value, self.num_buckets)


@dataclasses.dataclass(eq=True, frozen=True, kw_only=True)
class StackedTableSpec:
  """A stack of tables that share dim (after padding), optimizer, combiner."""

  stack_name: str
  stack_vocab_size: int
  stack_embedding_dim: int
  optimizer: OptimizerSpec
  combiner: str
  total_sample_count: int
  max_ids_per_partition: int = 256
  max_unique_ids_per_partition: int = 256
  activation_mem_bytes_limit: int = DEFAULT_ACTIVATION_MEM_BYTES_LIMIT
  suggested_coo_buffer_size_per_device: int | None = None
  quantization_config: QuantizationConfig | None = None


@dataclasses.dataclass(eq=True, unsafe_hash=True, kw_only=True)
class TableSpec:
  """One embedding table."""

  name: str
  vocabulary_size: int
  embedding_dim: int
  initializer: CallableTableInitializer = dataclasses.field(
      default=None, compare=False)
  optimizer: OptimizerSpec = dataclasses.field(
      default_factory=SGDOptimizerSpec)
  combiner: str = "sum"
  max_ids_per_partition: int = 256
  max_unique_ids_per_partition: int = 256
  suggested_coo_buffer_size_per_device: int | None = None
  quantization_config: QuantizationConfig | None = None

  _initialized: bool = dataclasses.field(
      init=False, default=False, compare=False)
  _stacked_table_spec: StackedTableSpec | None = dataclasses.field(
      default=None, compare=False)
  _setting_in_stack: TableSettingInStack | None = dataclasses.field(
      default=None, compare=False)

  def __setattr__(self, name: str, value: Any):
    allowed_after_stacking = ("_stacked_table_spec", "_setting_in_stack",
                              "stacked_table_spec", "setting_in_stack")
    fdo_params = ("max_ids_per_partition", "max_unique_ids_per_partition",
                  "suggested_coo_buffer_size_per_device")
    if (name not in allowed_after_stacking and
        getattr(self, "_initialized", False) and self.is_stacked()):
      if name in fdo_params:
        raise AttributeError(
            f"Cannot update parameter '{name}' on TableSpec '{self.name}' "
            "after it has been stacked. If you are trying to update FDO "
            "parameters like 'max_ids_per_partition', use "
            "embedding.update_preprocessing_parameters() to update the "
            "StackedTableSpec instead.")
      raise AttributeError(
          f"Cannot update parameter '{name}' on TableSpec '{self.name}' "
          "after it has been stacked.")
    super().__setattr__(name, value)

  @property
  def setting_in_stack(self) -> TableSettingInStack:
    assert self._setting_in_stack is not None
    return self._setting_in_stack

  @setting_in_stack.setter
  def setting_in_stack(self, v: TableSettingInStack) -> None:
    self._setting_in_stack = v

  @property
  def stacked_table_spec(self) -> StackedTableSpec:
    assert self._stacked_table_spec is not None, (
        f"Table {self.name} is not stacked.")
    return self._stacked_table_spec

  @stacked_table_spec.setter
  def stacked_table_spec(self, v: StackedTableSpec) -> None:
    self._stacked_table_spec = v

  def is_stacked(self) -> bool:
    return self._stacked_table_spec is not None

  def __post_init__(self):
    if self._setting_in_stack is None:
      self._setting_in_stack = TableSettingInStack(
          stack_name=self.name,
          padded_vocab_size=self.vocabulary_size,
          padded_embedding_dim=self.embedding_dim,
          row_offset_in_shard=0,
          shard_rotation=0,
      )
    object.__setattr__(self, "_initialized", True)


@dataclasses.dataclass(eq=True, unsafe_hash=True, kw_only=True)
class FeatureSpec:
  """One input feature: its table, input shape [batch, valency] and output
  shape [batch, embedding_dim]."""

  name: str
  table_spec: TableSpec
  input_shape: Sequence[int] = dataclasses.field(compare=False)
  output_shape: Sequence[int] = dataclasses.field(compare=False)
  _id_transformation: FeatureIdTransformation | None = dataclasses.field(
      default=None, compare=False)

  @property
  def id_transformation(self) -> FeatureIdTransformation:
    assert self._id_transformation is not None, self.name
    return self._id_transformation

  @id_transformation.setter
  def id_transformation(self, v: FeatureIdTransformation) -> None:
    self._id_transformation = v
