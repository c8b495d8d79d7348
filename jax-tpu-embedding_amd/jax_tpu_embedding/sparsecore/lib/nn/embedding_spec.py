"""Table / feature / stack specs (reference: lib/nn/embedding_spec.py).

The dataclasses keep the reference's field names, defaults and stacking
rules (``FeatureIdTransformation`` :918-938, ``TableSettingInStack``
:940-977, ``TableSpec`` :979-1118, ``FeatureSpec`` :1120-1166,
``StackedTableSpec`` :1169-1205, ``QuantizationConfig`` :1207-1223) so feature
specs written for the reference work unchanged. The optimizers are those of
the reference: SGD (:377-412), Adagrad (:415-460), Adam (:463-557),
AdagradMomentum (:560-649), FTRL (:652-741), LaProp (:744-830) and F2A
(:833-916), with the same hyperparameters, slot variables and defaults, and
the custom optimizer (:250-374) given by its update function.
Learning rates may be numbers, 0-d torch tensors or callables of the step.

Initializers are callables ``init(generator, shape)`` returning a float32
array; ``init_embedding_variables`` calls them with a ``torch.Generator`` on
the GPU. ``constant``, ``zeros`` and ``normal`` below cover the reference
defaults.
"""

from __future__ import annotations

import dataclasses
import inspect
from typing import Any, Callable, NamedTuple, Sequence

import numpy as np

from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad_momentum
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adam
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_f2a
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_ftrl
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_laprop
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_optimizer_grad

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


class F2ASlotVariables(NamedTuple):
  accumulator: Any
  local_step: Any


class AdamSlotVariables(NamedTuple):
  momentum: Any
  velocity: Any


class AdagradMomentumSlotVariables(NamedTuple):
  accumulator: Any
  momentum: Any


class FTRLSlotVariables(NamedTuple):
  accumulator: Any
  linear: Any


class LaPropSlotVariables(NamedTuple):
  mu: Any
  nu: Any


class CallablePlaceholder:
  """Stands in for a callable learning rate read back from a spec proto
  (embedding_spec.py:53-76): comparable by its tag, not callable."""

  def __init__(self, tag: str):
    self.tag = tag

  def __call__(self, *args, **kwargs):
    raise RuntimeError(
        f"CallablePlaceholder '{self.tag}' cannot be evaluated during model"
        " execution. It is intended only for spec inspection and table"
        " stacking.")

  def __eq__(self, other: object) -> bool:
    return isinstance(other, CallablePlaceholder) and self.tag == other.tag

  def __hash__(self) -> int:
    return hash(self.tag)

  def __repr__(self) -> str:
    return f"CallablePlaceholder({self.tag!r})"


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

  @classmethod
  def from_float_and_bool_params(cls, float_params: dict[str, float],
                                 bool_params: dict[str, bool],
                                 learning_rate: LearningRate):
    """The spec whose get_float_params / get_bool_params gave these
    values (embedding_spec.py:232-247)."""
    kwargs: dict[str, Any] = {"learning_rate": learning_rate}
    for p in cls._float_params:
      if p in float_params:
        kwargs[p] = float(float_params[p])
    for p in cls._bool_params:
      if p in bool_params:
        kwargs[p] = bool(bool_params[p])
    return cls(**kwargs)


class CustomOptimizerSpec(OptimizerSpec):
  """An optimizer given by its row-wise update (embedding_spec.py:250-374).

  `custom_computation_fn(gradient, table, *slots, *hyperparameters)` returns
  the new table, or (new table, *new slots); the hyperparameters are those of
  get_hyperparameters() (the learning rate). Alternatively `stablehlo` holds
  the update as a StableHLO module. Either is run per touched row by the
  tpu_sparse_dense_matmul_optimizer_grad primitive; see
  custom_optimizer_lowering for what the function may use.
  """

  def __init__(self, learning_rate: LearningRate = 0.001,
               custom_computation_fn: Callable[..., Any] | None = None,
               stablehlo: str | bytes | Any | None = None,
               slot_variable_initializers_tuple: tuple[
                   CallableTableInitializer, ...] = (),
               short_name_str: str = "custom"):
    super().__init__(learning_rate=learning_rate)
    self.custom_computation_fn = custom_computation_fn
    self.stablehlo = stablehlo
    self.slot_variable_initializers_tuple = slot_variable_initializers_tuple
    self.short_name_str = short_name_str

  def slot_variables_initializers(self) -> tuple:
    return self.slot_variable_initializers_tuple

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate), self.custom_computation_fn,
                 self.stablehlo, self.slot_variable_initializers_tuple,
                 self.short_name_str))

  def short_name(self) -> str:
    return self.short_name_str

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_optimizer_grad
            .tpu_sparse_dense_matmul_optimizer_grad_primitive)

  @classmethod
  def lower_to_stablehlo(cls, custom_computation_fn, embedding_dim: int = 1,
                         num_slot_variables: int = 0,
                         num_hyperparameters: int = 1,
                         min_value: float | None = None,
                         max_value: float | None = None) -> str:
    from jax_tpu_embedding.sparsecore.lib.nn import custom_optimizer_lowering  # pylint: disable=g-import-not-at-top

    return custom_optimizer_lowering.lower_to_stablehlo(
        custom_computation_fn, embedding_dim=embedding_dim,
        num_slot_variables=num_slot_variables,
        num_hyperparameters=num_hyperparameters, min_value=min_value,
        max_value=max_value)

  @classmethod
  def wrap_stablehlo_with_limits(cls, stablehlo, embedding_dim: int,
                                 num_slot_variables: int,
                                 num_hyperparameters: int,
                                 min_value: float | None = None,
                                 max_value: float | None = None) -> str:
    from jax_tpu_embedding.sparsecore.lib.nn import custom_optimizer_lowering  # pylint: disable=g-import-not-at-top

    return custom_optimizer_lowering.wrap_stablehlo_with_limits(
        stablehlo, embedding_dim=embedding_dim,
        num_slot_variables=num_slot_variables,
        num_hyperparameters=num_hyperparameters, min_value=min_value,
        max_value=max_value)


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


def _f32(x):
  return np.float32(x)


def _step_value(step) -> float:
  """The step as a number (0-d tensors are read back)."""
  if step is None:
    return 0.0
  if hasattr(step, "item"):
    return float(step.item())
  return float(step)


class AdamOptimizerSpec(OptimizerSpec):
  """Adam (Kingma et al., 2014) with the bias correction folded into the
  hyperparameters (embedding_spec.py:463-557)."""

  _float_params = ("beta_1", "beta_2", "epsilon")

  def __init__(self, learning_rate: LearningRate = 0.001,
               beta_1: float = 0.9, beta_2: float = 0.999,
               epsilon: float = 1e-8):
    super().__init__(learning_rate=learning_rate)
    self.beta_1 = beta_1
    self.beta_2 = beta_2
    self.epsilon = epsilon

  def slot_variables_initializers(self) -> tuple:
    return AdamSlotVariables(momentum=constant(0.0), velocity=constant(0.0))

  def get_hyperparameters(self, step=None) -> tuple:
    """(alpha_t, beta_1, beta_2, epsilon_hat) with
    alpha_t = lr * sqrt(1 - beta_2^t) / (1 - beta_1^t) and
    epsilon_hat = epsilon * sqrt(1 - beta_2^t), t = step + 1, in float32
    (embedding_spec.py:506-539)."""
    t = _step_value(step) + 1.0
    beta_1 = _f32(self.beta_1)
    beta_2 = _f32(self.beta_2)
    beta_1_t = np.power(beta_1, _f32(t))
    beta_2_t = np.power(beta_2, _f32(t))
    c_2 = np.sqrt(_f32(1.0) - beta_2_t)
    lr = self.get_learning_rate(step)
    if hasattr(lr, "data_ptr"):  # a 0-d torch tensor stays a tensor
      alpha_t = lr * float(c_2) / float(_f32(1.0) - beta_1_t)
    else:
      alpha_t = _f32(lr) * c_2 / (_f32(1.0) - beta_1_t)
    epsilon_hat = _f32(self.epsilon) * c_2
    return (alpha_t, beta_1, beta_2, epsilon_hat)

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate), self.beta_1, self.beta_2,
                 self.epsilon))

  def short_name(self) -> str:
    return "adam"

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_grad_with_adam
            .tpu_sparse_dense_matmul_grad_with_adam_primitive)


class AdagradMomentumOptimizerSpec(OptimizerSpec):
  """Adagrad with momentum (embedding_spec.py:560-649)."""

  _float_params = ("momentum", "beta2", "epsilon", "exponent",
                   "initial_accumulator_value", "initial_momentum_value")
  _bool_params = ("use_nesterov",)

  def __init__(self, learning_rate: LearningRate = 0.001,
               momentum: float = 0.9, beta2: float = 1.0,
               epsilon: float = 1e-10, exponent: float = 2.0,
               use_nesterov: bool = False,
               initial_accumulator_value: float = 0.1,
               initial_momentum_value: float = 0.0):
    super().__init__(learning_rate=learning_rate)
    self.momentum = momentum
    self.beta2 = beta2
    self.epsilon = epsilon
    self.exponent = exponent
    self.use_nesterov = use_nesterov
    self.initial_accumulator_value = initial_accumulator_value
    self.initial_momentum_value = initial_momentum_value

  def slot_variables_initializers(self) -> tuple:
    return AdagradMomentumSlotVariables(
        accumulator=constant(self.initial_accumulator_value),
        momentum=constant(self.initial_momentum_value))

  def get_hyperparameters(self, step=None) -> tuple:
    return (self.get_learning_rate(step), _f32(self.momentum),
            _f32(self.beta2), _f32(self.epsilon), _f32(self.exponent),
            np.bool_(self.use_nesterov))

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate), self.momentum, self.beta2,
                 self.epsilon, self.exponent, self.use_nesterov,
                 self.initial_accumulator_value,
                 self.initial_momentum_value))

  def short_name(self) -> str:
    return "adagrad_momentum"

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_grad_with_adagrad_momentum
            .tpu_sparse_dense_matmul_grad_with_adagrad_momentum_primitive)


class FTRLOptimizerSpec(OptimizerSpec):
  """Follow The Regularized Leader (embedding_spec.py:652-741)."""

  _float_params = ("learning_rate_power", "l1_regularization_strength",
                   "l2_regularization_strength", "beta",
                   "initial_accumulator_value", "initial_linear_value")
  _bool_params = ("multiply_linear_by_learning_rate",)

  def __init__(self, learning_rate: LearningRate = 0.01,
               learning_rate_power: float = -0.5,
               l1_regularization_strength: float = 0.0,
               l2_regularization_strength: float = 0.0, beta: float = 0.0,
               initial_accumulator_value: float = 0.1,
               initial_linear_value: float = 0.0,
               multiply_linear_by_learning_rate: bool = False):
    super().__init__(learning_rate=learning_rate)
    self.learning_rate_power = learning_rate_power
    self.l1_regularization_strength = l1_regularization_strength
    self.l2_regularization_strength = l2_regularization_strength
    self.beta = beta
    self.initial_accumulator_value = initial_accumulator_value
    self.initial_linear_value = initial_linear_value
    self.multiply_linear_by_learning_rate = multiply_linear_by_learning_rate

  def slot_variables_initializers(self) -> tuple:
    return FTRLSlotVariables(
        accumulator=constant(self.initial_accumulator_value),
        linear=constant(self.initial_linear_value))

  def get_hyperparameters(self, step=None) -> tuple:
    return (self.get_learning_rate(step), _f32(self.learning_rate_power),
            _f32(self.l1_regularization_strength),
            _f32(self.l2_regularization_strength), _f32(self.beta))

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate), self.learning_rate_power,
                 self.l1_regularization_strength,
                 self.l2_regularization_strength, self.beta,
                 self.initial_accumulator_value, self.initial_linear_value,
                 self.multiply_linear_by_learning_rate))

  def short_name(self) -> str:
    return "ftrl"

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_grad_with_ftrl
            .tpu_sparse_dense_matmul_grad_with_ftrl_primitive)


class LaPropOptimizerSpec(OptimizerSpec):
  """LaProp (arXiv:2002.04839; embedding_spec.py:744-830)."""

  _float_params = ("b1", "b2", "eps", "initial_slot_value")

  def __init__(self, learning_rate: LearningRate = 0.001, b1: float = 0.9,
               b2: float = 0.95, eps: float = 1e-30,
               rms_clip_threshold: float | None = None,
               initial_slot_value: float = 0.0):
    super().__init__(learning_rate=learning_rate)
    self.b1 = b1
    self.b2 = b2
    self.eps = eps
    if rms_clip_threshold is not None:
      raise ValueError(
          "rms_clip_threshold is not yet supported in LaProp optimizer.")
    self.initial_slot_value = initial_slot_value

  def slot_variables_initializers(self) -> tuple:
    return LaPropSlotVariables(mu=constant(self.initial_slot_value),
                               nu=constant(self.initial_slot_value))

  def get_decay_rate(self, step=None):
    """b2 without a step, else b2 (1 - b2^step) / (1 - b2^(step + 1)) in
    float32 (embedding_spec.py:788-800)."""
    b2 = _f32(self.b2)
    if step is None:
      return b2
    st = _f32(_step_value(step))
    return _f32(b2 * (_f32(1.0) - np.power(b2, st)) /
                (_f32(1.0) - np.power(b2, st + _f32(1.0))))

  def get_hyperparameters(self, step=None) -> tuple:
    return (self.get_learning_rate(step), _f32(self.b1),
            self.get_decay_rate(step), _f32(self.eps))

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate), self.b1, self.b2, self.eps,
                 self.initial_slot_value))

  def short_name(self) -> str:
    return "laprop"

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_grad_with_laprop
            .tpu_sparse_dense_matmul_grad_with_laprop_primitive)


class F2AOptimizerSpec(OptimizerSpec):
  """Frequency-aware Adagrad (embedding_spec.py:833-916)."""

  _float_params = ("rho", "initial_accumulator_value",
                   "initial_local_step_value", "l1_regularization_strength",
                   "l2_regularization_strength", "max_lr_multiplier")

  def __init__(self, learning_rate: LearningRate = 0.01, rho: float = 0.5,
               initial_accumulator_value: float = 0.1,
               initial_local_step_value: float = 0.0,
               l1_regularization_strength: float = 0.0,
               l2_regularization_strength: float = 0.0,
               max_lr_multiplier: float = 1e6):
    super().__init__(learning_rate=learning_rate)
    self.rho = rho
    self.initial_accumulator_value = initial_accumulator_value
    self.initial_local_step_value = initial_local_step_value
    self.l1_regularization_strength = l1_regularization_strength
    self.l2_regularization_strength = l2_regularization_strength
    self.max_lr_multiplier = max_lr_multiplier

  def slot_variables_initializers(self) -> tuple:
    return F2ASlotVariables(
        accumulator=constant(self.initial_accumulator_value),
        local_step=constant(self.initial_local_step_value))

  def get_hyperparameters(self, step=None) -> tuple:
    if step is None:
      step = 0
    return (self.get_learning_rate(step), _f32(self.rho),
            _f32(self.l1_regularization_strength),
            _f32(self.l2_regularization_strength),
            _f32(self.max_lr_multiplier), _f32(_step_value(step)))

  def __hash__(self) -> int:
    return hash((_hashable(self.learning_rate), self.rho,
                 self.initial_accumulator_value,
                 self.initial_local_step_value,
                 self.l1_regularization_strength,
                 self.l2_regularization_strength, self.max_lr_multiplier))

  def short_name(self) -> str:
    return "f2a"

  def get_optimizer_primitive(self):
    return (sparse_dense_matmul_grad_with_f2a
            .tpu_sparse_dense_matmul_grad_with_f2a_primitive)


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

  def replace(self, **changes) -> "StackedTableSpec":
    """A copy with `changes` (flax struct.PyTreeNode.replace of the
    reference's spec, embedding_spec.py:1169)."""
    return dataclasses.replace(self, **changes)


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
