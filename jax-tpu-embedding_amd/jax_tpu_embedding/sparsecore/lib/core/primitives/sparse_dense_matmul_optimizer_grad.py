"""Primitive tpu_sparse_dense_matmul_optimizer_grad: backward + a custom update.

Same operands and attributes as the reference primitive
(``lib/core/primitives/sparse_dense_matmul_optimizer_grad.py:66-138``
abstract eval, ``:147-260`` lowering to
``SparseDenseMatmulGradOpWithOptimizerUpdate``): the CSR, the activation
gradients, then ``num_hyperparameters`` hyperparameters (float32 scalars or
1-element vectors) and the embedding variables (the table first, then its
slot variables, each rank 2), and ``stablehlo``, the row-wise update as a
StableHLO module whose ``@main`` takes (gradient, table, *slots,
*hyperparameters) and returns (table, *slots). ``bind`` returns the updated
variables, updated in place when they are float32 CUDA tensors.

The module is read into an element-wise program
(``custom_optimizer_lowering.parse_stablehlo``; an ``UpdateProgram`` is
accepted as well) and run by ``scemb_sparse_dense_matmul_grad_with_optimizer``
with ``SCEMB_OPTIMIZER_CUSTOM``: the gradient of every touched row is summed
as for the built-in optimizers, then the program updates the row once. At
most 2 slot variables, 8 hyperparameters and 48 operations.
"""

from __future__ import annotations

import functools

import numpy as np

from jax_tpu_embedding.sparsecore import _native
from jax_tpu_embedding.sparsecore.lib.core.primitives import _optimizer
from jax_tpu_embedding.sparsecore.lib.core.primitives import utils
from jax_tpu_embedding.sparsecore.lib.nn import custom_optimizer_lowering


@functools.lru_cache(maxsize=64)
def _program_from_text(text: str, num_slots: int, num_hyper: int):
  prog = custom_optimizer_lowering.parse_stablehlo(text, num_slots, num_hyper)
  return _native.update_program(prog.compile())


def program_struct(stablehlo, num_slots: int, num_hyper: int):
  """The kernel's program for a StableHLO module (str or bytes) or an
  UpdateProgram."""
  if isinstance(stablehlo, custom_optimizer_lowering.UpdateProgram):
    if (stablehlo.num_slots, stablehlo.num_hyperparameters) != (num_slots,
                                                                num_hyper):
      raise ValueError("the update program was traced for "
                       f"{stablehlo.num_slots} slot variables and "
                       f"{stablehlo.num_hyperparameters} hyperparameters")
    return _native.update_program(stablehlo.compile())
  if isinstance(stablehlo, bytes):
    stablehlo = stablehlo.decode("utf-8")
  if not isinstance(stablehlo, str):
    raise ValueError(
        "stablehlo must be a string, bytes, or ir.Module, got"
        f" {type(stablehlo)}")
  return _program_from_text(stablehlo, num_slots, num_hyper)


def _check_hyperparameter(param):
  # Python and numpy float scalars become float32 operands, as jax's dtype
  # canonicalisation (64-bit types off) makes them before this check.
  if isinstance(param, (float, int, np.floating)) and not isinstance(
      param, bool):
    return
  dtype = getattr(param, "dtype", None)
  if dtype is None or str(dtype).split(".")[-1] != "float32":
    raise ValueError(f"hyperparameters must be float32, got {dtype}")
  shape = tuple(getattr(param, "shape", ()))
  if shape not in ((), (1,)):
    raise ValueError(
        f"hyperparameters must be scalars or 1D of size 1, got {shape}")


def _impl(lhs_row_pointers, lhs_local_embedding_ids, lhs_local_sample_ids,
          lhs_gains, num_minibatches_per_physical_sparse_core,
          activations_grad, *hyperparams_and_embedding_vars,
          num_hyperparameters: int, stablehlo, max_ids_per_partition: int,
          max_unique_ids_per_partition: int,
          computation_name: str = "sparse_dense_matmul_optimizer_grad",
          sharding_strategy: int = 1, enable_minibatching: bool = False,
          **kwargs):
  hyper = hyperparams_and_embedding_vars[:num_hyperparameters]
  variables = hyperparams_and_embedding_vars[num_hyperparameters:]
  if not variables:
    raise ValueError("At least one embedding variable must be passed.")
  for param in hyper:
    _check_hyperparameter(param)
  for var in variables:
    if len(getattr(var, "shape", ())) != 2:
      raise ValueError(
          f"embedding variables must have rank 2, got {tuple(var.shape)}")
  _optimizer.check_same_shape(
      variables[0], [(f"slot {i}", v) for i, v in enumerate(variables[1:])],
      lambda *shapes: "embedding variables must have equal shapes, got "
      f"{shapes}")
  if len(variables) - 1 > 2:
    raise NotImplementedError(
        "custom optimizers with more than 2 slot variables are not "
        "supported")
  program = program_struct(stablehlo, len(variables) - 1, len(hyper))
  hyper = tuple(np.float32(h) if isinstance(h, (float, int, np.floating))
                else h.reshape(()) for h in hyper)
  return _optimizer.apply(
      _native.OPTIMIZER_CUSTOM, lhs_row_pointers, lhs_local_embedding_ids,
      lhs_local_sample_ids, lhs_gains,
      num_minibatches_per_physical_sparse_core, variables[0],
      tuple(variables[1:]), activations_grad, hyper,
      max_ids_per_partition=max_ids_per_partition,
      max_unique_ids_per_partition=max_unique_ids_per_partition,
      computation_name=computation_name, sharding_strategy=sharding_strategy,
      enable_minibatching=enable_minibatching, program=program, **kwargs)


tpu_sparse_dense_matmul_optimizer_grad_primitive = utils.Primitive(
    "sparse_dense_matmul_optimizer_grad_primitive", _impl)
tpu_sparse_dense_matmul_optimizer_grad_primitive.multiple_results = True
