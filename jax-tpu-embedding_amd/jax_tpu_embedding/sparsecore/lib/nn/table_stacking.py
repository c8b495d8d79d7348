"""Table and feature stacking (reference: lib/nn/table_stacking.py).

Stacking concatenates tables of equal padded dim / optimizer / combiner along
the vocabulary (each table's vocab padded to a multiple of 8 * NS, NS = number
of SparseCores; table shards rotated by ``rotation``), and feature stacking
concatenates the batches of all features that read a stack. The arithmetic is
the reference's, because the CSR ids it produces index the stacked buffer:
  padded dim / vocab        round_up_dim_and_vocab_size (:355-378)
  groups                    _group_tables_for_stacking (:381-396) and the
                            activation-memory split (:399-498)
  settings in stack         compute_table_to_setting_in_stack (:570-613)
  feature transformation    _stack_feature_specs (:648-754): row_offset =
                            samples before the feature, col_offset =
                            row_offset_in_shard * NS, col_shift = rotation
  physical rows             compute_physical_row_ids (:1229-1255)
  stack / shard of values   stack_and_shard_tables (:144-221) and its inverse
                            unshard_and_unstack_tables (:226-311)
  from a spec proto         stack_and_shard_feature_tables (:1080-1226),
                            unstack_and_unshard_stacked_tables (:963-1077),
                            get_row_ids_in_stacked_table(s) (:1258-1330)
Table values here are numpy arrays or torch tensors.
"""

from __future__ import annotations

import collections
import hashlib
import logging
from typing import Callable, Mapping, Sequence

import numpy as np

from jax_tpu_embedding.sparsecore import _tree
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec

LimitsCallable = Callable[[str, int], int]
DEFAULT_ACTIVATION_MEM_BYTES_LIMIT = (
    embedding_spec.DEFAULT_ACTIVATION_MEM_BYTES_LIMIT)


def _next_largest_multiple(value: int, multiple: int) -> int:
  return ((value + multiple - 1) // multiple) * multiple


def get_default_limits(name: str, batch_size: int) -> int:
  del name, batch_size
  return 256


def round_up_dim_and_vocab_size(tables: Mapping[str,
                                                embedding_spec.TableSpec],
                                num_sc: int):
  """Padded dims (multiple of 8) and vocab sizes (multiple of 8 * num_sc)."""
  dims = {n: _next_largest_multiple(s.embedding_dim, 8)
          for n, s in tables.items()}
  vocabs = {n: _next_largest_multiple(s.vocabulary_size, 8 * num_sc)
            for n, s in tables.items()}
  return dims, vocabs


def _group_tables_for_stacking(num_sc, tables):
  dims, _ = round_up_dim_and_vocab_size(tables, num_sc)
  groups = collections.defaultdict(list)
  for name, dim in dims.items():
    spec = tables[name]
    groups[(dim, spec.optimizer, spec.combiner,
            spec.quantization_config)].append(name)
  return list(groups.values())


def _activation_mem_bytes(num_sc, tables, features):
  counts = collections.defaultdict(int)
  for f in features:
    counts[f.table_spec.name] += int(np.prod(f.output_shape[:-1]) // num_sc)
  dims, _ = round_up_dim_and_vocab_size(tables, num_sc)
  return {n: dims[n] * counts[n] * 4 for n in tables}


def _split_groups_by_memory_limit(groups, mem, limit):
  out = []
  for group in groups:
    split: list[list[str]] = []
    for name in group:
      for cand in split:
        if sum(mem[c] for c in cand) + mem[name] <= limit:
          cand.append(name)
          break
      else:
        split.append([name])
    out.extend(split)
  return out


def _is_stacked_already(table: embedding_spec.TableSpec) -> bool:
  s = table._setting_in_stack  # pylint: disable=protected-access
  return s is not None and s.stack_name != table.name


def _verify_stack_tables(stack_name, table_names, features, tables):
  for t in table_names:
    if _is_stacked_already(tables[t]):
      raise ValueError(f"Table {t} is already stacked in group "
                       f"{tables[t].setting_in_stack.stack_name}.")
  for f in features:
    if (_is_stacked_already(f.table_spec) and
        f.table_spec.setting_in_stack.stack_name == stack_name):
      raise ValueError(f"Cannot use stack name {stack_name} since it's "
                       "already used.")
  for t, n in collections.Counter(table_names).items():
    if n > 1:
      raise ValueError(f"Table {t} is repeated in group {stack_name}.")
  first = tables[table_names[0]]
  if not all(tables[t].optimizer == first.optimizer for t in table_names):
    raise ValueError(f"Tables {table_names} in group {stack_name} have "
                     "different optimizers.")
  if not all(tables[t].combiner == first.combiner for t in table_names):
    raise ValueError(f"Tables {table_names} in group {stack_name} have "
                     "different combiners.")
  if not all(tables[t].quantization_config == first.quantization_config
             for t in table_names):
    raise ValueError(f"Tables {table_names} in group {stack_name} have "
                     "different quantization configs.")


def compute_table_to_setting_in_stack(stack_name: str,
                                      table_names: Sequence[str],
                                      padded_embedding_dim: int,
                                      table_to_padded_vocab_size: Mapping[str,
                                                                          int],
                                      num_shards: int, rotation: int):
  """Row offset in shard (cumulative shard rows) and shard rotation."""
  out = {}
  row_offset_in_shard = 0
  shard_rotation = 0
  for name in table_names:
    if name not in table_to_padded_vocab_size:
      raise ValueError(f"Padded vocab size for Table {name} is missing.")
    out[name] = embedding_spec.TableSettingInStack(
        stack_name=stack_name,
        padded_vocab_size=table_to_padded_vocab_size[name],
        padded_embedding_dim=padded_embedding_dim,
        row_offset_in_shard=row_offset_in_shard,
        shard_rotation=shard_rotation)
    row_offset_in_shard += table_to_padded_vocab_size[name] // num_shards
    shard_rotation = (shard_rotation + rotation) % num_shards
  return out


def _get_stack_name(table_names: Sequence[str],
                    use_short_stack_names: bool = True,
                    max_original_display_length: int = 50,
                    hash_length: int = 12) -> str:
  name = "_".join(table_names)
  if not use_short_stack_names:
    return name
  short = name[:max_original_display_length]
  if len(name) > max_original_display_length:
    short += "..." + hashlib.sha256(name.encode("utf-8")).hexdigest()[
        :hash_length]
  return short


def _stack_feature_specs(*, stack_name, features, table_names,
                         padded_embedding_dim, table_to_padded_vocab_size,
                         global_device_count, num_sc_per_device, rotation,
                         stack_to_max_ids_per_partition,
                         stack_to_max_unique_ids_per_partition,
                         activation_mem_bytes_limit):
  ns = global_device_count * num_sc_per_device
  settings = compute_table_to_setting_in_stack(
      stack_name, table_names, padded_embedding_dim,
      table_to_padded_vocab_size, ns, rotation)
  leaves = _tree.tree_leaves(features)
  stacked_features = [f for f in leaves if f.table_spec.name in table_names]
  row_offsets = {}
  sample_count = 0
  for f in stacked_features:
    row_offsets[f.name] = sample_count
    sample_count += int(np.prod(f.output_shape[:-1]))
  if len(table_names) == 1:
    ts = next(f.table_spec for f in leaves
              if f.table_spec.name == table_names[0])
    max_ids, max_unique = ts.max_ids_per_partition, \
        ts.max_unique_ids_per_partition
  else:
    logging.warning(
        "Stacking multiple tables together: %s. Per-table limits are "
        "replaced by the stack defaults; use "
        "embedding.update_preprocessing_parameters to override them.",
        table_names)
    max_ids = stack_to_max_ids_per_partition(stack_name, sample_count)
    max_unique = stack_to_max_unique_ids_per_partition(stack_name,
                                                       sample_count)
  first = stacked_features[0].table_spec
  stacked = embedding_spec.StackedTableSpec(
      stack_name=stack_name,
      stack_vocab_size=sum(table_to_padded_vocab_size[t] for t in table_names),
      stack_embedding_dim=padded_embedding_dim,
      optimizer=first.optimizer,
      combiner=first.combiner,
      total_sample_count=sample_count,
      max_ids_per_partition=max_ids,
      max_unique_ids_per_partition=max_unique,
      activation_mem_bytes_limit=activation_mem_bytes_limit,
      quantization_config=first.quantization_config)
  for f in leaves:
    if f.table_spec.name not in table_names:
      continue
    setting = settings[f.table_spec.name]
    f.table_spec.stacked_table_spec = stacked
    f.table_spec.setting_in_stack = setting
    f.id_transformation = embedding_spec.FeatureIdTransformation(
        row_offset=row_offsets[f.name],
        col_offset=setting.row_offset_in_shard * ns,
        col_shift=setting.shard_rotation)


def stack_tables(features, table_names: Sequence[str],
                 global_device_count: int, num_sc_per_device: int,
                 rotation: int | None = None,
                 stack_to_max_ids_per_partition: LimitsCallable = (
                     get_default_limits),
                 stack_to_max_unique_ids_per_partition: LimitsCallable = (
                     get_default_limits),
                 stack_name: str | None = None,
                 fail_on_excess_padding: bool = False, *,
                 activation_mem_bytes_limit: int = (
                     DEFAULT_ACTIVATION_MEM_BYTES_LIMIT)) -> None:
  """Stacks `table_names` into one stacked table; updates specs in place."""
  if not stack_name:
    stack_name = _get_stack_name(table_names)
  leaves = _tree.tree_leaves(features)
  tables = {f.table_spec.name: f.table_spec for f in leaves
            if f.table_spec.name in table_names}
  ns = num_sc_per_device * global_device_count
  dims, vocabs = round_up_dim_and_vocab_size(tables, ns)
  padded_dim = max(dims.values())
  if not all(dims[t] == padded_dim for t in table_names):
    excess = sum((padded_dim - dims[t]) * vocabs[t] for t in table_names)
    msg = (f"Excess padding detected for stacked table {stack_name}: "
           f"{excess} values.")
    if fail_on_excess_padding:
      raise ValueError(msg)
    logging.warning(msg)
  _verify_stack_tables(stack_name, list(table_names), leaves, tables)
  rotation = rotation if rotation is not None else num_sc_per_device
  _stack_feature_specs(
      stack_name=stack_name, features=features, table_names=list(table_names),
      padded_embedding_dim=padded_dim, table_to_padded_vocab_size=vocabs,
      global_device_count=global_device_count,
      num_sc_per_device=num_sc_per_device, rotation=rotation,
      stack_to_max_ids_per_partition=stack_to_max_ids_per_partition,
      stack_to_max_unique_ids_per_partition=(
          stack_to_max_unique_ids_per_partition),
      activation_mem_bytes_limit=activation_mem_bytes_limit)


def auto_stack_tables(features, global_device_count: int,
                      num_sc_per_device: int, rotation: int | None = None,
                      stack_to_max_ids_per_partition: LimitsCallable = (
                          get_default_limits),
                      stack_to_max_unique_ids_per_partition: LimitsCallable = (
                          get_default_limits), *,
                      use_short_stack_names: bool = True,
                      activation_mem_bytes_limit: int | None = (
                          DEFAULT_ACTIVATION_MEM_BYTES_LIMIT)) -> None:
  """Stacks all compatible tables (grouped and split by activation memory)."""
  if activation_mem_bytes_limit is None:
    activation_mem_bytes_limit = DEFAULT_ACTIVATION_MEM_BYTES_LIMIT
  leaves = _tree.tree_leaves(features)
  tables = {f.table_spec.name: f.table_spec for f in leaves}
  ns = num_sc_per_device * global_device_count
  groups = _group_tables_for_stacking(ns, tables)
  mem = _activation_mem_bytes(ns, tables, leaves)
  groups = _split_groups_by_memory_limit(groups, mem,
                                         activation_mem_bytes_limit)
  if set(tables) != {t for g in groups for t in g}:
    raise ValueError("Table names are not grouped correctly.")
  for group in groups:
    stack_tables(
        features, group, global_device_count, num_sc_per_device, rotation,
        stack_to_max_ids_per_partition, stack_to_max_unique_ids_per_partition,
        stack_name=_get_stack_name(group, use_short_stack_names),
        fail_on_excess_padding=False,
        activation_mem_bytes_limit=activation_mem_bytes_limit)


def get_table_stacks(table_specs) -> dict[str, list[embedding_spec.TableSpec]]:
  out = collections.defaultdict(list)
  for t in _tree.tree_leaves(table_specs):
    name = (t.stacked_table_spec.stack_name if t.is_stacked() else t.name)
    out[name].append(t)
  return dict(out)


def compute_physical_row_ids(num_sparse_cores: int, stack_vocab_size: int,
                             shard_rotation: int, row_offset_in_shard: int,
                             row_ids):
  """Physical row of logical row ids of a table in its stacked buffer."""
  shard_size = stack_vocab_size // num_sparse_cores
  shard_id = (row_ids % num_sparse_cores + shard_rotation) % num_sparse_cores
  sharded_row = row_ids // num_sparse_cores + row_offset_in_shard
  return shard_id * shard_size + sharded_row


def get_row_ids_in_stacked_table(stack_table_spec, table_spec,
                                 row_ids) -> list[int]:
  """Rows of the stacked buffer holding rows `row_ids` of one table
  (StackedTableSpecProto, TableSpecProto)."""
  out = []
  for row_id in row_ids:
    if row_id >= table_spec.vocab_size:
      raise ValueError(f"{row_id} exceeds available vocabulary size "
                       f"[{table_spec.vocab_size}].")
    out.append(compute_physical_row_ids(
        stack_table_spec.num_sparsecores, stack_table_spec.stack_vocab_size,
        table_spec.shard_rotation, table_spec.row_offset_in_shard, row_id))
  return out


def get_row_ids_in_stacked_tables(embedding_spec_proto,
                                  row_ids: Mapping) -> dict[str, list[int]]:
  """Stacked-buffer rows of the tables' rows in `row_ids` (keyed by table
  name), grouped by stack name in the proto's table order."""
  out: dict[str, list[int]] = collections.defaultdict(list)
  for stack in embedding_spec_proto.stacked_table_specs:
    for table in stack.table_specs:
      if table.table_name in row_ids:
        out[stack.stack_name].extend(get_row_ids_in_stacked_table(
            stack, table, row_ids[table.table_name]))
  return out


# ---------------------------------------------------------------------------
# Table values.
# ---------------------------------------------------------------------------


def _is_torch(x) -> bool:
  return type(x).__module__.startswith("torch")


def _stack_one(stacked, spec: embedding_spec.TableSpec, values, num_shards,
               pad_value):
  padded_vocab = _next_largest_multiple(spec.vocabulary_size, 8 * num_shards)
  dim = stacked.shape[-1]
  per_shard = padded_vocab // num_shards
  setting = spec.setting_in_stack
  if _is_torch(values):
    import torch  # pylint: disable=g-import-not-at-top

    padded = torch.full((padded_vocab, dim), pad_value, dtype=torch.float32,
                        device=values.device)
    padded[:spec.vocabulary_size, :spec.embedding_dim] = values.reshape(
        spec.vocabulary_size, -1)[:, :spec.embedding_dim]
    sharded = padded.reshape(per_shard, num_shards, dim).transpose(0, 1)
    sharded = torch.roll(sharded, setting.shard_rotation, dims=0)
  else:
    padded = np.full((padded_vocab, dim), pad_value, np.float32)
    padded[:spec.vocabulary_size, :spec.embedding_dim] = np.asarray(
        values, np.float32).reshape(spec.vocabulary_size, -1)[
            :, :spec.embedding_dim]
    sharded = np.swapaxes(padded.reshape(per_shard, num_shards, dim), 0, 1)
    sharded = np.roll(sharded, setting.shard_rotation, axis=0)
  r = setting.row_offset_in_shard
  stacked[:, r:r + per_shard, :] = sharded
  return stacked


def stack_and_shard_tables(table_specs, tables, num_shards: int,
                           pad_value: float = float("nan")) -> dict:
  """Builds each stacked buffer [num_shards, vocab_per_shard, dim] from the
  unstacked tables; reshape to [vocab, dim] for the lookup (a device's
  shard is the whole buffer on one GPU)."""
  spec_leaves = _tree.tree_leaves(table_specs)
  value_leaves = _tree.tree_leaves(tables)
  by_name = {s.name: v for s, v in zip(spec_leaves, value_leaves)}
  stacks: dict[str, list] = collections.defaultdict(list)
  for s in spec_leaves:
    name = s.stacked_table_spec.stack_name if s.is_stacked() else s.name
    stacks[name].append(s)
  out = {}
  for name, specs in stacks.items():
    first = specs[0]
    if first.is_stacked():
      vocab = first.stacked_table_spec.stack_vocab_size
      dim = first.stacked_table_spec.stack_embedding_dim
    else:
      vocab = _next_largest_multiple(first.vocabulary_size, 8 * num_shards)
      dim = _next_largest_multiple(first.embedding_dim, 8)
    sample = by_name[first.name]
    if _is_torch(sample):
      import torch  # pylint: disable=g-import-not-at-top

      buf = torch.zeros((num_shards, vocab // num_shards, dim),
                        dtype=torch.float32, device=sample.device)
    else:
      buf = np.zeros((num_shards, vocab // num_shards, dim), np.float32)
    for s in specs:
      buf = _stack_one(buf, s, by_name[s.name], num_shards, pad_value)
    out[name] = buf
  return out


def _unshard_one(stacked_3d, row_offset_in_shard: int, per_shard: int,
                 shard_rotation: int, vocab_size: int, embedding_dim: int):
  """One table [vocab, dim] out of a stacked buffer viewed as
  [num_shards, rows_per_shard, dim]: its rows of every shard, shards turned
  back by the rotation, rows interleaved back (row i of shard s is logical
  row i * num_shards + s), padding dropped."""
  dim = stacked_3d.shape[-1]
  r = row_offset_in_shard
  part = stacked_3d[:, r:r + per_shard, :]
  if _is_torch(part):
    import torch  # pylint: disable=g-import-not-at-top

    part = torch.roll(part, -shard_rotation, dims=0)
    part = part.transpose(0, 1).reshape(-1, dim)
  else:
    part = np.roll(part, -shard_rotation, axis=0)
    part = np.swapaxes(part, 0, 1).reshape(-1, dim)
  return part[:vocab_size, :embedding_dim]


def unshard_and_unstack_tables(table_specs, stacked_tables: Mapping,
                               num_shards: int):
  """Recovers each table [vocab, dim] from its stacked buffer."""

  def one(spec):
    name = spec.stacked_table_spec.stack_name if spec.is_stacked() else \
        spec.name
    st = stacked_tables[name]
    dim = st.shape[-1]
    per_shard = _next_largest_multiple(spec.vocabulary_size,
                                       8 * num_shards) // num_shards
    setting = spec.setting_in_stack
    return _unshard_one(st.reshape(num_shards, -1, dim),
                        setting.row_offset_in_shard, per_shard,
                        setting.shard_rotation, spec.vocabulary_size,
                        spec.embedding_dim)

  return _tree.tree_map(one, table_specs)


# ---------------------------------------------------------------------------
# The same, driven by an EmbeddingSpecProto (checkpoint conversion).
# ---------------------------------------------------------------------------


def _unstack_and_unshard_stacked_table(stacked_table, stacked_table_spec,
                                       donate: bool = False) -> dict:
  """Tables of one stack, by name, from its stacked buffer [vocab, dim].
  `donate` is accepted for the reference's signature; the buffer is left
  to the caller."""
  del donate
  ns = stacked_table_spec.num_sparsecores
  st = stacked_table.reshape(ns, -1, stacked_table_spec.stack_embedding_dim)
  out = {}
  for t in stacked_table_spec.table_specs:
    out[t.table_name] = _unshard_one(st, t.row_offset_in_shard,
                                     t.padded_vocab_size // ns,
                                     t.shard_rotation, t.vocab_size,
                                     t.embedding_dim)
  return out


def unstack_and_unshard_stacked_tables(stacked_tables: Mapping,
                                       embedding_specs,
                                       donate: bool = False) -> dict:
  """Every table of an EmbeddingSpecProto, by name, from the stacked
  buffers keyed by stack name."""
  out = {}
  for spec in embedding_specs.stacked_table_specs:
    table = stacked_tables.get(spec.stack_name)
    if table is None:
      raise ValueError(f"Stacked table '{spec.stack_name}' not found in "
                       "`stacked_tables`.")
    out.update(_unstack_and_unshard_stacked_table(table, spec, donate))
  return out


def _shard_one(table, padded_vocab_size: int, padded_embedding_dim: int,
               num_shards: int, shard_rotation: int):
  """[num_shards, padded_vocab / num_shards, dim] block of one table:
  zero padding, then logical row i to shard i % num_shards (row
  i // num_shards), shards rotated by `shard_rotation`."""
  rows, cols = table.shape
  per_shard = padded_vocab_size // num_shards
  if _is_torch(table):
    import torch  # pylint: disable=g-import-not-at-top

    padded = torch.zeros((padded_vocab_size, padded_embedding_dim),
                         dtype=table.dtype, device=table.device)
    padded[:rows, :cols] = table
    block = padded.reshape(per_shard, num_shards, -1).transpose(0, 1)
    return torch.roll(block, shard_rotation, dims=0)
  padded = np.zeros((padded_vocab_size, padded_embedding_dim),
                    np.asarray(table).dtype)
  padded[:rows, :cols] = np.asarray(table)
  block = np.swapaxes(padded.reshape(per_shard, num_shards, -1), 0, 1)
  return np.roll(block, shard_rotation, axis=0)


def stack_and_shard_feature_tables(feature_tables: Mapping, embedding_specs,
                                   delete_input: bool = False) -> dict:
  """The stacked buffer [stack_vocab, dim] of every stack of an
  EmbeddingSpecProto from the unstacked tables keyed by table name.
  `delete_input` is accepted for the reference's signature; the inputs are
  left to the caller."""
  del delete_input
  out = {}
  for spec in embedding_specs.stacked_table_specs:
    blocks = []
    for t in spec.table_specs:
      table = feature_tables.get(t.table_name)
      if table is None:
        raise ValueError(f"{t.table_name}' not found in `feature_tables`.")
      if spec.stack_embedding_dim != t.padded_embedding_dim:
        raise ValueError(
            f"Embedding dim of table_spec {t.table_name} is "
            f"{t.padded_embedding_dim} but the stacked table embedding dim "
            f"is {spec.stack_embedding_dim}.")
      blocks.append(_shard_one(table, t.padded_vocab_size,
                               t.padded_embedding_dim, spec.num_sparsecores,
                               t.shard_rotation))
    if blocks and _is_torch(blocks[0]):
      import torch  # pylint: disable=g-import-not-at-top

      stacked = torch.cat(blocks, dim=1)
    else:
      stacked = np.concatenate(blocks, axis=1)
    out[spec.stack_name] = stacked.reshape(-1, spec.stack_embedding_dim)
  return out
