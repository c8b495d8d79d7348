"""Spec <-> proto conversion (reference: lib/nn/embedding_proto_utils.py).

`create_proto_from_feature_specs` records the stacked layout of prepared
feature specs in an `EmbeddingSpecProto` (embedding_proto_utils.py:199-283):
one `StackedTableSpecProto` per stack, in the order the stacks first occur in
the flattened features, each with its tables in first-occurrence order and
each table with its features. The unstack / restack helpers of
`table_stacking` read it, so stacked tables saved by the reference can be
unstacked here and the other way round.

Optimizers map to `OptimizerSpecProto` by type (:56-109); LaProp has no enum
value in the schema and becomes CUSTOM, as in the reference. A callable
learning rate is stored as a tag (:112-131) and comes back as a
`CallablePlaceholder`.
"""

from __future__ import annotations

import collections
from typing import Any

from jax_tpu_embedding.sparsecore import _tree
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from jax_tpu_embedding.sparsecore.lib.proto import embedding_spec_pb2
from jax_tpu_embedding.sparsecore.utils import utils

_OPT = embedding_spec_pb2.OptimizerSpecProto

_OPTIMIZER_TYPE_TO_CLASS = {
    _OPT.SGD: embedding_spec.SGDOptimizerSpec,
    _OPT.ADAGRAD: embedding_spec.AdagradOptimizerSpec,
    _OPT.ADAM: embedding_spec.AdamOptimizerSpec,
    _OPT.FTRL: embedding_spec.FTRLOptimizerSpec,
    _OPT.F2A: embedding_spec.F2AOptimizerSpec,
    _OPT.ADAGRAD_MOMENTUM: embedding_spec.AdagradMomentumOptimizerSpec,
}
_OPTIMIZER_CLASS_TO_TYPE = {c: t for t, c in _OPTIMIZER_TYPE_TO_CLASS.items()}


def _get_num_sc_per_device(num_sc_per_device: int | None) -> int:
  if num_sc_per_device is None:
    return utils.num_sparsecores_per_device()
  if num_sc_per_device not in utils.NUM_SC_PER_DEVICE_MAP.values():
    raise ValueError(f"Invalid num_sc_per_device: {num_sc_per_device}")
  return num_sc_per_device


def get_optimizer_class(optimizer_type) -> type | None:
  """The OptimizerSpec class of a proto optimizer type, or None."""
  return _OPTIMIZER_TYPE_TO_CLASS.get(optimizer_type)


def get_optimizer_type(optimizer_class) -> int:
  """The proto optimizer type of an OptimizerSpec class (CUSTOM if none)."""
  return _OPTIMIZER_CLASS_TO_TYPE.get(optimizer_class, _OPT.CUSTOM)


def _extract_learning_rate_tag(learning_rate) -> str | None:
  if not callable(learning_rate) or isinstance(learning_rate, (int, float)):
    return None
  tag = getattr(learning_rate, "tag", None)
  if tag:
    return str(tag)
  name = getattr(learning_rate, "__qualname__",
                 getattr(learning_rate, "__name__", ""))
  if name and name != "<lambda>":
    module = getattr(learning_rate, "__module__", "")
    return f"{module}.{name}" if module else name
  return f"{type(learning_rate).__name__}_{id(learning_rate)}"


def optimizer_spec_to_proto(opt):
  """OptimizerSpecProto of an optimizer spec (None stays None)."""
  if opt is None:
    return None
  kwargs: dict[str, Any] = {}
  tag = _extract_learning_rate_tag(opt.learning_rate)
  if tag:
    kwargs["learning_rate_tag"] = tag
  elif isinstance(opt.learning_rate, (int, float)):
    kwargs["learning_rate"] = float(opt.learning_rate)
  opt_type = get_optimizer_type(type(opt))
  custom = opt_type == _OPT.CUSTOM
  return _OPT(type=opt_type,
              float_params={} if custom else opt.get_float_params(),
              bool_params={} if custom else opt.get_bool_params(),
              **kwargs)


def proto_to_optimizer_spec(proto):
  """The optimizer spec of an OptimizerSpecProto; SGD for None or unknown
  types (embedding_proto_utils.py:168-196)."""
  if proto is None:
    return embedding_spec.SGDOptimizerSpec(learning_rate=0.0)
  if proto.WhichOneof("learning_rate_spec") == "learning_rate_tag":
    lr = embedding_spec.CallablePlaceholder(proto.learning_rate_tag)
  else:
    lr = proto.learning_rate
  cls = get_optimizer_class(proto.type)
  if cls is None:
    return embedding_spec.SGDOptimizerSpec(learning_rate=lr)
  return cls.from_float_and_bool_params(dict(proto.float_params),
                                        dict(proto.bool_params),
                                        learning_rate=lr)


def create_proto_from_feature_specs(feature_specs,
                                    global_device_count: int | None,
                                    num_sparsecore_per_device: int | None = None):
  """EmbeddingSpecProto of prepared (stacked) feature specs."""
  if global_device_count is None:
    global_device_count = 1
  num_sc = _get_num_sc_per_device(num_sparsecore_per_device)
  stacks: dict[str, Any] = {}
  tables: dict[str, dict[str, Any]] = collections.defaultdict(dict)
  for feature in _tree.tree_leaves(feature_specs):
    stacked = feature.table_spec.stacked_table_spec
    setting = feature.table_spec.setting_in_stack
    stack_name = stacked.stack_name
    table_name = feature.table_spec.name
    if stack_name not in stacks:
      stacks[stack_name] = embedding_spec_pb2.StackedTableSpecProto(
          stack_name=stack_name,
          stack_vocab_size=stacked.stack_vocab_size,
          stack_embedding_dim=stacked.stack_embedding_dim,
          total_sample_count=stacked.total_sample_count,
          max_ids_per_partition=stacked.max_ids_per_partition,
          num_sparsecores=num_sc * global_device_count,
          max_unique_ids_per_partition=stacked.max_unique_ids_per_partition,
          activation_mem_bytes_limit=stacked.activation_mem_bytes_limit)
    if table_name not in tables[stack_name]:
      tables[stack_name][table_name] = embedding_spec_pb2.TableSpecProto(
          table_name=table_name,
          vocab_size=feature.table_spec.vocabulary_size,
          embedding_dim=feature.table_spec.embedding_dim,
          padded_vocab_size=setting.padded_vocab_size,
          padded_embedding_dim=setting.padded_embedding_dim,
          row_offset_in_shard=setting.row_offset_in_shard,
          shard_rotation=setting.shard_rotation,
          combiner=feature.table_spec.combiner,
          optimizer=optimizer_spec_to_proto(feature.table_spec.optimizer))
    tables[stack_name][table_name].feature_specs.append(
        embedding_spec_pb2.FeatureSpecProto(
            feature_name=feature.name,
            row_offset=feature.id_transformation.row_offset,
            col_offset=feature.id_transformation.col_offset,
            col_shift=feature.id_transformation.col_shift,
            input_shape=list(feature.input_shape),
            output_shape=list(feature.output_shape)))
  for stack_name, specs in tables.items():
    stacks[stack_name].table_specs.extend(specs.values())
  return embedding_spec_pb2.EmbeddingSpecProto(
      stacked_table_specs=list(stacks.values()))
