"""Protocol-buffer messages of the embedding layout.

The schema is the reference's `lib/proto/embedding_spec.proto` (messages
FeatureSpecProto, OptimizerSpecProto, TableSpecProto, StackedTableSpecProto,
EmbeddingSpecProto): same package, field names, numbers and types, so that a
serialized spec moves between the reference and this build (checkpoints keep
one beside the stacked tables). No `protoc` runs here: the file descriptor is
assembled with `descriptor_pb2` and the message classes come from the
protobuf runtime.
"""

from __future__ import annotations

from google.protobuf import descriptor_pb2
from google.protobuf import descriptor_pool
from google.protobuf import message_factory

_PACKAGE = "third_party.py.jax_tpu_embedding.sparsecore_lib_proto"
_FILE = "jax_tpu_embedding/sparsecore/lib/proto/embedding_spec.proto"

_F = descriptor_pb2.FieldDescriptorProto
_SCALARS = {
    "string": _F.TYPE_STRING,
    "int64": _F.TYPE_INT64,
    "float": _F.TYPE_FLOAT,
    "bool": _F.TYPE_BOOL,
}


def _field(msg, name, number, kind, repeated=False, oneof=None,
           proto3_optional=False):
  f = msg.field.add()
  f.name = name
  f.number = number
  f.label = _F.LABEL_REPEATED if repeated else _F.LABEL_OPTIONAL
  if kind in _SCALARS:
    f.type = _SCALARS[kind]
  elif kind.startswith("enum:"):
    f.type = _F.TYPE_ENUM
    f.type_name = f".{_PACKAGE}.{kind[5:]}"
  else:
    f.type = _F.TYPE_MESSAGE
    f.type_name = f".{_PACKAGE}.{kind}"
  if oneof is not None:
    f.oneof_index = oneof
  if proto3_optional:
    f.proto3_optional = True
  return f


def _map_field(msg, name, number, value_kind, entry_name):
  entry = msg.nested_type.add()
  entry.name = entry_name
  entry.options.map_entry = True
  _field(entry, "key", 1, "string")
  _field(entry, "value", 2, value_kind)
  _field(msg, name, number, f"{msg.name}.{entry_name}", repeated=True)


def _file_descriptor() -> descriptor_pb2.FileDescriptorProto:
  fd = descriptor_pb2.FileDescriptorProto()
  fd.name = _FILE
  fd.package = _PACKAGE
  fd.syntax = "proto3"
  fd.options.java_multiple_files = True

  feat = fd.message_type.add()
  feat.name = "FeatureSpecProto"
  _field(feat, "feature_name", 1, "string")
  _field(feat, "input_shape", 2, "int64", repeated=True)
  _field(feat, "output_shape", 3, "int64", repeated=True)
  _field(feat, "row_offset", 4, "int64")
  _field(feat, "col_offset", 5, "int64")
  _field(feat, "col_shift", 6, "int64")

  opt = fd.message_type.add()
  opt.name = "OptimizerSpecProto"
  enum = opt.enum_type.add()
  enum.name = "OptimizerType"
  for i, n in enumerate(("OPTIMIZER_TYPE_UNSPECIFIED", "SGD", "ADAGRAD",
                         "ADAM", "FTRL", "F2A", "ADAGRAD_MOMENTUM",
                         "CUSTOM")):
    v = enum.value.add()
    v.name = n
    v.number = i
  opt.oneof_decl.add().name = "learning_rate_spec"
  _field(opt, "type", 1, "enum:OptimizerSpecProto.OptimizerType")
  _field(opt, "learning_rate", 2, "float", oneof=0)
  _field(opt, "learning_rate_tag", 3, "string", oneof=0)
  _map_field(opt, "float_params", 4, "float", "FloatParamsEntry")
  _map_field(opt, "bool_params", 5, "bool", "BoolParamsEntry")

  table = fd.message_type.add()
  table.name = "TableSpecProto"
  _field(table, "table_name", 1, "string")
  _field(table, "vocab_size", 2, "int64")
  _field(table, "embedding_dim", 3, "int64")
  _field(table, "max_ids_per_partition", 5, "int64")
  _field(table, "max_unique_ids_per_partition", 6, "int64")
  _field(table, "padded_vocab_size", 7, "int64")
  _field(table, "padded_embedding_dim", 8, "int64")
  _field(table, "row_offset_in_shard", 9, "int64")
  _field(table, "shard_rotation", 10, "int64")
  _field(table, "feature_specs", 11, "FeatureSpecProto", repeated=True)
  _field(table, "combiner", 12, "string")
  _field(table, "optimizer", 13, "OptimizerSpecProto")

  stacked = fd.message_type.add()
  stacked.name = "StackedTableSpecProto"
  _field(stacked, "stack_name", 1, "string")
  _field(stacked, "stack_vocab_size", 2, "int64")
  _field(stacked, "stack_embedding_dim", 3, "int64")
  _field(stacked, "total_sample_count", 6, "int64")
  _field(stacked, "max_ids_per_partition", 7, "int64")
  _field(stacked, "max_unique_ids_per_partition", 8, "int64")
  _field(stacked, "num_sparsecores", 9, "int64")
  _field(stacked, "table_specs", 10, "TableSpecProto", repeated=True)
  # proto3 `optional`: a synthetic one-field oneof.
  stacked.oneof_decl.add().name = "_activation_mem_bytes_limit"
  _field(stacked, "activation_mem_bytes_limit", 11, "int64", oneof=0,
         proto3_optional=True)

  spec = fd.message_type.add()
  spec.name = "EmbeddingSpecProto"
  _field(spec, "stacked_table_specs", 1, "StackedTableSpecProto",
         repeated=True)
  return fd


def _load():
  pool = descriptor_pool.DescriptorPool()
  file_desc = pool.Add(_file_descriptor())
  del file_desc
  out = {}
  for name in ("FeatureSpecProto", "OptimizerSpecProto", "TableSpecProto",
               "StackedTableSpecProto", "EmbeddingSpecProto"):
    desc = pool.FindMessageTypeByName(f"{_PACKAGE}.{name}")
    out[name] = message_factory.GetMessageClass(desc)
  return out


_CLASSES = _load()
FeatureSpecProto = _CLASSES["FeatureSpecProto"]
OptimizerSpecProto = _CLASSES["OptimizerSpecProto"]
TableSpecProto = _CLASSES["TableSpecProto"]
StackedTableSpecProto = _CLASSES["StackedTableSpecProto"]
EmbeddingSpecProto = _CLASSES["EmbeddingSpecProto"]
