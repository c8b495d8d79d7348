"""Table stacking and the stacked layout against the reference's own tests.

Transcribed from the reference (paths under jax_tpu_embedding/sparsecore/):
  lib/nn/tests/table_stacking_test.py  ComputePhysicalRowIdsTest (:28-59),
      no stacking (:67-83), auto stacking (:85-217, :219-282, :284-359 memory
      limit, :361-494 Adagrad), manual stacking (:496-612, :614-694), errors
      (:696-800), _split_groups_by_memory_limit (:802-893), unstack
      (:895-1143), stack and shard (:1145-1379), stacked row ids
      (:1381-1644), quantization configs (:1646-1832);
  lib/nn/tests/embedding_test.py  feature stacking (:233-286), manual
      settings (:170-231, :288-380), spec proto (:1037-1165).
The reference runs these on TPUs with 2 or 4 SparseCores per device and
1-4 devices; here the SparseCore count S and device count G are parameters,
covering the reference's combinations (S in {2, 4}) and S = 1, the MI355X
setting. Where an expectation is a literal of the reference test, it is kept
literal, and where a literal holds only for some S x G the case is limited
to those.

Expected stacked arrays come from `_reference_stacked_shards`, a brute-force
restatement of the reference test helper
`create_per_device_sharded_stacked_tables` (lib/nn/tests/test_utils.py:
133-169): logical row r of the i-th table goes to shard
(r % T + i * rotation) % T at row r // T of that table's block (T = G * S).
"""

import numpy as np
import pytest
from google.protobuf import text_format

from jax_tpu_embedding.sparsecore.lib.nn import embedding
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from jax_tpu_embedding.sparsecore.lib.nn import table_stacking
from jax_tpu_embedding.sparsecore.lib.proto import embedding_spec_pb2

SG = [(1, 1), (1, 2), (1, 4), (2, 1), (2, 2), (2, 4), (4, 1), (4, 2), (4, 4)]


def _round_up(x, m):
  return (x + m - 1) // m * m


def _row_ids(shape, offset=0):
  """test_utils.row_id_initializer: row i holds offset + i."""
  return np.broadcast_to(
      np.arange(offset, offset + shape[0], dtype=np.float32)[:, None],
      shape).copy()


def _reference_stacked_shards(tables, num_devices, num_sc, rotation):
  """[num_devices, rows per device, dim] stacked buffer, built row by row."""
  rotation = num_sc if rotation is None else rotation
  t = num_devices * num_sc
  dim = tables[0].shape[1]
  per = [tab.shape[0] // t for tab in tables]
  out = np.zeros((t, sum(per), dim), np.float32)
  offset = 0
  for i, tab in enumerate(tables):
    for r in range(tab.shape[0]):
      out[(r % t + i * rotation) % t, offset + r // t] = tab[r]
    offset += per[i]
  return out.reshape(num_devices, -1, dim)


def _table(name, vocab, dim, optimizer=None, **kw):
  return embedding_spec.TableSpec(
      vocabulary_size=vocab, embedding_dim=dim, initializer=None,
      optimizer=optimizer or embedding_spec.SGDOptimizerSpec(),
      combiner="sum", name=name, max_ids_per_partition=16,
      max_unique_ids_per_partition=16, **kw)


def _feature(name, table, batch=16):
  return embedding_spec.FeatureSpec(
      table_spec=table, input_shape=(batch, 1),
      output_shape=(batch, table.embedding_dim), name=name)


# --- ComputePhysicalRowIdsTest (table_stacking_test.py:28-59) ---------------


def test_compute_physical_row_ids_scalar():
  # 4 SparseCores, stack vocab 100, rotation 1, row offset in shard 10.
  assert table_stacking.compute_physical_row_ids(4, 100, 1, 10, 5) == 61


def test_compute_physical_row_ids_array():
  got = table_stacking.compute_physical_row_ids(
      4, 100, 1, 10, np.array([0, 1, 2, 3, 4]))
  np.testing.assert_array_equal(got, [35, 60, 85, 10, 36])


# --- TableStackingTest ------------------------------------------------------


def test_no_stacking():
  t = _table("table_a", 64, 12)
  s = t.setting_in_stack
  assert (s.stack_name, s.padded_vocab_size, s.padded_embedding_dim,
          s.row_offset_in_shard, s.shard_rotation) == ("table_a", 64, 12, 0, 0)


def _three_features(optimizer_a=None, optimizer_b=None):
  a = _table("table_a", 64, 12, optimizer_a)
  b = _table("table_b", 120, 10, optimizer_b)
  return [_feature("feature_spec_a", a), _feature("feature_spec_b", b),
          _feature("feature_spec_c", b)]


@pytest.mark.parametrize("num_sc,devices", SG)
@pytest.mark.parametrize("adagrad", [False, True])
def test_auto_stack_two_tables(num_sc, devices, adagrad):
  opt = (lambda: embedding_spec.AdagradOptimizerSpec(
      learning_rate=0.5, initial_accumulator_value=1.0)) if adagrad else (
          embedding_spec.SGDOptimizerSpec)
  features = _three_features(opt(), opt())
  table_stacking.auto_stack_tables(features, global_device_count=devices,
                                   num_sc_per_device=num_sc)
  fa, fb, fc = features
  ns = devices * num_sc
  pa = _round_up(64, 8 * ns)
  pb = _round_up(120, 8 * ns)
  sa, sb = fa.table_spec.setting_in_stack, fb.table_spec.setting_in_stack
  assert sa.stack_name == sb.stack_name == "table_a_table_b"
  assert (sa.padded_vocab_size, sa.padded_embedding_dim,
          sa.row_offset_in_shard) == (pa, 16, 0)
  assert (fa.id_transformation.row_offset, fa.id_transformation.col_offset,
          fa.id_transformation.col_shift) == (0, 0, 0)
  assert (sb.padded_vocab_size, sb.padded_embedding_dim,
          sb.row_offset_in_shard) == (pb, 16, pa // ns)
  assert fb.id_transformation.row_offset == 16
  assert fb.id_transformation.col_offset == sb.row_offset_in_shard * ns
  assert fc.id_transformation.row_offset == 32
  assert fc.id_transformation.col_offset == sb.row_offset_in_shard * ns


@pytest.mark.parametrize("short", [True, False])
def test_auto_stack_short_stack_names(short):
  a = _table("table_foo_bar_transaction_history_log", 128, 12)
  b = _table("table_foo_bar_customer_profile_data", 128, 10)
  features = [_feature("feature_spec_a", a), _feature("feature_spec_b", b)]
  table_stacking.auto_stack_tables(features, global_device_count=1,
                                   num_sc_per_device=4,
                                   use_short_stack_names=short)
  expected = ("table_foo_bar_transaction_history_log_table_foo_ba..."
              "0618d69c6704" if short else
              "table_foo_bar_transaction_history_log_"
              "table_foo_bar_customer_profile_data")
  assert features[0].table_spec.setting_in_stack.stack_name == expected
  assert features[1].table_spec.setting_in_stack.stack_name == expected


# The reference runs this on 2 devices of a TPU with 2 or 4 SparseCores.
@pytest.mark.parametrize("num_sc", [2, 4])
@pytest.mark.parametrize("limit,stacks", [(128, 2), (1024, 1)])
def test_auto_stack_with_mem_limit(num_sc, limit, stacks):
  features = _three_features()
  table_stacking.auto_stack_tables(features, global_device_count=2,
                                   num_sc_per_device=num_sc,
                                   activation_mem_bytes_limit=limit)
  fa, fb, _ = features
  if stacks == 1:
    assert fa.table_spec.setting_in_stack.stack_name == "table_a_table_b"
    assert fb.table_spec.setting_in_stack.stack_name == "table_a_table_b"
  else:
    assert fa.table_spec.setting_in_stack.stack_name == "table_a"
    assert fb.table_spec.setting_in_stack.stack_name == "table_b"


@pytest.mark.parametrize("num_sc,devices", SG)
def test_manual_stacking(num_sc, devices):
  a = _table("table_a", 64, 12, embedding_spec.SGDOptimizerSpec(0.5))
  b = _table("table_b", 120, 10)
  c = _table("table_c", 120, 16)
  features = [_feature("feature_spec_a", a), _feature("feature_spec_b", b),
              _feature("feature_spec_c", c)]
  table_stacking.stack_tables(features, ["table_a"],
                              global_device_count=devices,
                              num_sc_per_device=num_sc)

  def limits(name, batch_size):
    del name
    return int(batch_size * 0.8)

  table_stacking.stack_tables(features, ["table_c", "table_b"],
                              global_device_count=devices,
                              stack_to_max_ids_per_partition=limits,
                              stack_to_max_unique_ids_per_partition=limits,
                              num_sc_per_device=num_sc)
  fa, fb, fc = features
  assert fa.table_spec.setting_in_stack.stack_name == "table_a"
  assert fa.table_spec.setting_in_stack.padded_embedding_dim == 16
  assert fb.table_spec.setting_in_stack.stack_name == "table_c_table_b"
  assert fc.table_spec.setting_in_stack.stack_name == "table_c_table_b"
  ns = devices * num_sc
  assert fb.table_spec.setting_in_stack.padded_vocab_size == _round_up(
      120, 8 * ns)
  assert fb.table_spec.setting_in_stack.padded_embedding_dim == 16
  assert fb.table_spec.setting_in_stack.shard_rotation == num_sc % ns
  # Two features of 16 samples: int(32 * 0.8).
  assert fb.table_spec.stacked_table_spec.max_ids_per_partition == 25
  assert fb.table_spec.stacked_table_spec.max_unique_ids_per_partition == 25


@pytest.mark.parametrize("num_sc,devices", SG)
def test_manual_stacking_reuse_table_name(num_sc, devices):
  a = _table("A", 64, 12, embedding_spec.SGDOptimizerSpec(0.5))
  b = _table("B", 120, 10, embedding_spec.SGDOptimizerSpec(0.5))
  c = _table("C", 120, 10, embedding_spec.SGDOptimizerSpec(0.5))
  features = [_feature("feature_a", a), _feature("feature_b", b),
              _feature("feature_c", c)]
  table_stacking.stack_tables(features, ("A", "B"),
                              global_device_count=devices,
                              num_sc_per_device=num_sc,
                              stack_name="custom_stack")
  with pytest.raises(ValueError, match="custom_stack.*already used.*"):
    table_stacking.stack_tables(features, ("C",),
                                global_device_count=devices,
                                num_sc_per_device=num_sc,
                                stack_name="custom_stack")


def test_manual_stacking_not_same_optimizer():
  a = _table("A", 64, 12, embedding_spec.SGDOptimizerSpec(0.5))
  b = _table("B", 120, 10)
  features = [_feature("feature_a", a), _feature("feature_b", b)]
  with pytest.raises(ValueError, match=".*different optimizers.*"):
    table_stacking.stack_tables(features, ("A", "B"), global_device_count=1,
                                num_sc_per_device=1)


def test_manual_stacking_overlapping_stacks():
  a = _table("A", 64, 12)
  b = _table("B", 120, 10)
  c = _table("C", 120, 16)

  def fresh():
    return [_feature("feature_a", a), _feature("feature_b", b),
            _feature("feature_c", c)]

  with pytest.raises(ValueError, match="Table A is repeated in group"):
    table_stacking.stack_tables(fresh(), ("A", "B", "A"),
                                global_device_count=1, num_sc_per_device=4)
  table_stacking.stack_tables(fresh(), ("A", "B"), global_device_count=1,
                              num_sc_per_device=4)
  with pytest.raises(ValueError, match="Table B is already stacked."):
    table_stacking.stack_tables(fresh(), ("C", "B"), global_device_count=1,
                                num_sc_per_device=4)


@pytest.mark.parametrize("groups,mem,limit,expected", [
    ([["a", "b", "c"]], {"a": 10, "b": 20, "c": 30}, 100, [["a", "b", "c"]]),
    ([["a", "b", "c"]], {"a": 10, "b": 20, "c": 30}, 30, [["a", "b"], ["c"]]),
    ([["a", "b", "c"]], {"a": 10, "b": 20, "c": 30}, 35, [["a", "b"], ["c"]]),
    ([["a", "b", "c", "d"]], {"a": 10, "b": 10, "c": 10, "d": 10}, 25,
     [["a", "b"], ["c", "d"]]),
    ([["a"], ["b", "c"]], {"a": 10, "b": 20, "c": 30}, 35,
     [["a"], ["b"], ["c"]]),
    ([["a", "b"], ["c", "d"]], {"a": 10, "b": 20, "c": 5, "d": 5}, 30,
     [["a", "b"], ["c", "d"]]),
    ([["a", "b", "c"]], {"a": 60, "b": 60, "c": 60}, 50,
     [["a"], ["b"], ["c"]]),
    ([["a", "b", "c"]], {"a": 10, "b": 20, "c": 30}, 60, [["a", "b", "c"]]),
    ([["a", "b", "c"]], {"a": 10, "b": 20, "c": 30}, 40, [["a", "b"], ["c"]]),
    ([["a", "b"], ["c"]], {"a": 10, "b": 20, "c": 30}, 30,
     [["a", "b"], ["c"]]),
    ([["a", "b"], ["c", "d"]], {"a": 10, "b": 15, "c": 20, "d": 25}, 30,
     [["a", "b"], ["c"], ["d"]]),
    ([], {"a": 10}, 100, []),
])
def test_split_groups_by_memory_limit(groups, mem, limit, expected):
  assert table_stacking._split_groups_by_memory_limit(  # pylint: disable=protected-access
      groups, mem, limit) == expected


# --- Unstacking and stacking of values (table_stacking_test.py:895-1379) ----


def _unstack_case(num_sc, devices, rotation):
  batch = 16
  a = embedding_spec.TableSpec(vocabulary_size=32, embedding_dim=14,
                               initializer=None, name="table_a")
  b = embedding_spec.TableSpec(vocabulary_size=128, embedding_dim=14,
                               initializer=None, name="table_b")
  c = embedding_spec.TableSpec(vocabulary_size=256, embedding_dim=32,
                               initializer=None, name="table_c")
  fa = embedding_spec.FeatureSpec(table_spec=a, input_shape=[batch, 1],
                                  output_shape=[batch, 14], name="feature_a")
  fb = embedding_spec.FeatureSpec(table_spec=b, input_shape=[batch, 1],
                                  output_shape=[batch, 14], name="feature_b")
  fc = embedding_spec.FeatureSpec(table_spec=c, input_shape=[batch, 1],
                                  output_shape=[batch, 14], name="feature_c")
  specs_ab, specs_c = [fa, fb], [fc]
  table_stacking.auto_stack_tables(specs_ab, num_sc_per_device=num_sc,
                                   global_device_count=devices,
                                   rotation=rotation)
  table_stacking.auto_stack_tables(specs_c, num_sc_per_device=num_sc,
                                   global_device_count=devices,
                                   rotation=rotation)
  ta = _row_ids((a.setting_in_stack.padded_vocab_size,
                 a.setting_in_stack.padded_embedding_dim), 0)
  tb = _row_ids((b.setting_in_stack.padded_vocab_size,
                 b.setting_in_stack.padded_embedding_dim), 1000)
  tc = _row_ids((c.setting_in_stack.padded_vocab_size,
                 c.setting_in_stack.padded_embedding_dim), 0)
  var_ab = _reference_stacked_shards([ta, tb], devices, num_sc,
                                     rotation).reshape(-1, 16)
  var_c = _reference_stacked_shards([tc], devices, num_sc,
                                    rotation).reshape(-1, 32)
  return specs_ab, specs_c, (ta, tb, tc), (var_ab, var_c)


@pytest.mark.parametrize("num_sc,devices", SG)
@pytest.mark.parametrize("rotation", [None, 0, 2, 4, -1])
def test_unshard_and_unstack_stacked_table(num_sc, devices, rotation):
  specs_ab, specs_c, (ta, tb, tc), (var_ab, var_c) = _unstack_case(
      num_sc, devices, rotation)
  proto = embedding.create_proto_from_feature_specs(
      specs_ab, global_device_count=devices,
      num_sparsecore_per_device=num_sc)
  ret = table_stacking._unstack_and_unshard_stacked_table(  # pylint: disable=protected-access
      var_ab, proto.stacked_table_specs[0], donate=False)
  np.testing.assert_array_equal(ret["table_a"], ta[:32, :14])
  np.testing.assert_array_equal(ret["table_b"], tb[:128, :14])

  proto = embedding.create_proto_from_feature_specs(
      specs_ab + specs_c, global_device_count=devices,
      num_sparsecore_per_device=num_sc)
  ret = table_stacking.unstack_and_unshard_stacked_tables(
      {proto.stacked_table_specs[0].stack_name: var_ab,
       proto.stacked_table_specs[1].stack_name: var_c}, proto)
  np.testing.assert_array_equal(ret["table_a"], ta[:32, :14])
  np.testing.assert_array_equal(ret["table_b"], tb[:128, :14])
  np.testing.assert_array_equal(ret["table_c"], tc[:256, :32])

  # The spec-based inverse and the forward stacking agree with it too.
  tables = table_stacking.unshard_and_unstack_tables(
      {"table_a": specs_ab[0].table_spec, "table_b": specs_ab[1].table_spec},
      {"table_a_table_b": var_ab}, devices * num_sc)
  np.testing.assert_array_equal(tables["table_a"], ta[:32, :14])
  np.testing.assert_array_equal(tables["table_b"], tb[:128, :14])
  stacked = table_stacking.stack_and_shard_tables(
      {"table_a": specs_ab[0].table_spec, "table_b": specs_ab[1].table_spec},
      {"table_a": ta[:32, :14], "table_b": tb[:128, :14]}, devices * num_sc,
      pad_value=0.0)
  expected = _reference_stacked_shards(
      [np.pad(ta[:32, :14], ((0, ta.shape[0] - 32), (0, 2))),
       np.pad(tb[:128, :14], ((0, tb.shape[0] - 128), (0, 2)))],
      devices, num_sc, rotation).reshape(-1, 16)
  np.testing.assert_array_equal(
      stacked["table_a_table_b"].reshape(-1, 16), expected)


def test_unstack_missing_stack_raises():
  specs_ab, _, _, _ = _unstack_case(4, 1, None)
  proto = embedding.create_proto_from_feature_specs(
      specs_ab, global_device_count=1, num_sparsecore_per_device=4)
  with pytest.raises(ValueError, match="not found in `stacked_tables`"):
    table_stacking.unstack_and_unshard_stacked_tables({}, proto)


@pytest.mark.parametrize("num_sc,devices", SG)
@pytest.mark.parametrize("use_torch", [False, True])
def test_stacking_and_sharding_table(num_sc, devices, use_torch):
  batch = 16
  a = embedding_spec.TableSpec(vocabulary_size=64, embedding_dim=14,
                               initializer=None, name="table_a")
  b = embedding_spec.TableSpec(vocabulary_size=192, embedding_dim=14,
                               initializer=None, name="table_b")
  c = embedding_spec.TableSpec(vocabulary_size=120, embedding_dim=30,
                               initializer=None, name="table_c")
  specs_ab = [
      embedding_spec.FeatureSpec(table_spec=a, input_shape=[batch, 1],
                                 output_shape=[batch, 14], name="feature_a"),
      embedding_spec.FeatureSpec(table_spec=b, input_shape=[batch, 1],
                                 output_shape=[batch, 14], name="feature_b")]
  specs_c = [embedding_spec.FeatureSpec(table_spec=c, input_shape=[batch, 1],
                                        output_shape=[batch, 14],
                                        name="feature_c")]
  table_stacking.auto_stack_tables(specs_ab, num_sc_per_device=num_sc,
                                   global_device_count=devices)
  table_stacking.auto_stack_tables(specs_c, num_sc_per_device=num_sc,
                                   global_device_count=devices)
  ta, tb, tc = _row_ids((64, 14), 10), _row_ids((192, 14), 100), _row_ids(
      (120, 30), 1000)

  def pad(x, spec):
    s = spec.setting_in_stack
    return np.pad(x, ((0, s.padded_vocab_size - x.shape[0]),
                      (0, s.padded_embedding_dim - x.shape[1])))

  expected_ab = _reference_stacked_shards(
      [pad(ta, a), pad(tb, b)], devices, num_sc,
      b.setting_in_stack.shard_rotation).reshape(-1, 16)
  expected_c = _reference_stacked_shards([pad(tc, c)], devices, num_sc,
                                         0).reshape(-1, 32)
  proto = embedding.create_proto_from_feature_specs(
      specs_ab + specs_c, global_device_count=devices,
      num_sparsecore_per_device=num_sc)
  inputs = {"table_a": ta, "table_b": tb, "table_c": tc}
  if use_torch:
    import torch  # pylint: disable=g-import-not-at-top

    inputs = {k: torch.from_numpy(v) for k, v in inputs.items()}
  stacked = table_stacking.stack_and_shard_feature_tables(inputs, proto)
  got_ab = stacked[proto.stacked_table_specs[0].stack_name]
  got_c = stacked[proto.stacked_table_specs[1].stack_name]
  if use_torch:
    got_ab, got_c = got_ab.numpy(), got_c.numpy()
  np.testing.assert_array_equal(got_ab, expected_ab)
  np.testing.assert_array_equal(got_c, expected_c)


def _three_table_specs(num_sc, devices):
  specs = []
  for name, vocab, dim in (("table_a", 64, 4), ("table_b", 192, 5),
                           ("table_c", 224, 6)):
    t = embedding_spec.TableSpec(vocabulary_size=vocab, embedding_dim=dim,
                                 initializer=None, name=name)
    specs.append(embedding_spec.FeatureSpec(
        table_spec=t, input_shape=[16, 1], output_shape=[16, dim],
        name=name.replace("table", "feature")))
  table_stacking.auto_stack_tables(specs, num_sc_per_device=num_sc,
                                   global_device_count=devices)
  proto = embedding.create_proto_from_feature_specs(
      specs, global_device_count=devices, num_sparsecore_per_device=num_sc)
  return specs, proto


@pytest.mark.parametrize("num_sc,devices", SG)
def test_get_stacked_row_ids(num_sc, devices):
  specs, proto = _three_table_specs(num_sc, devices)
  tables = {f.table_spec.name: _row_ids(
      (f.table_spec.vocabulary_size, f.table_spec.embedding_dim), off)
            for f, off in zip(specs, (10, 100, 1000))}
  stacked = table_stacking.stack_and_shard_feature_tables(tables, proto)
  for stack in proto.stacked_table_specs:
    for t in stack.table_specs:
      rows = table_stacking.get_row_ids_in_stacked_table(
          stack, t, list(range(t.vocab_size)))
      for i in range(t.vocab_size):
        np.testing.assert_array_equal(
            stacked[stack.stack_name][rows[i]][:t.embedding_dim],
            tables[t.table_name][i])
  with pytest.raises(ValueError, match="exceeds available vocabulary size"):
    t0 = proto.stacked_table_specs[0].table_specs[0]
    table_stacking.get_row_ids_in_stacked_table(
        proto.stacked_table_specs[0], t0, [t0.vocab_size])


@pytest.mark.parametrize("num_sc,devices", SG)
def test_get_row_ids_in_stacked_tables(num_sc, devices):
  specs, proto = _three_table_specs(num_sc, devices)
  row_ids = {f.table_spec.name: list(range(f.table_spec.vocabulary_size))
             for f in specs}
  got = table_stacking.get_row_ids_in_stacked_tables(proto, row_ids)
  for stack in proto.stacked_table_specs:
    expected = []
    for t in stack.table_specs:
      if t.table_name in row_ids:
        expected.extend(table_stacking.get_row_ids_in_stacked_table(
            stack, t, row_ids[t.table_name]))
    assert got[stack.stack_name] == expected


def test_auto_stack_tables_with_quantization_config():
  q = embedding_spec.QuantizationConfig(min_value=-5.0, max_value=5.0,
                                        num_buckets=256)
  a = _table("table_a", 64, 12, quantization_config=q)
  b = _table("table_b", 120, 10, quantization_config=q)
  features = [_feature("feature_spec_a", a), _feature("feature_spec_b", b)]
  table_stacking.auto_stack_tables(features, global_device_count=1,
                                   num_sc_per_device=4)
  assert features[0].table_spec.stacked_table_spec.quantization_config == q
  assert features[1].table_spec.stacked_table_spec.quantization_config == q
  assert features[0].table_spec.setting_in_stack.stack_name == (
      "table_a_table_b")


def test_auto_stack_tables_different_quantization_configs_split():
  q1 = embedding_spec.QuantizationConfig(min_value=-5.0, max_value=5.0,
                                         num_buckets=256)
  q2 = embedding_spec.QuantizationConfig(min_value=-2.0, max_value=2.0,
                                         num_buckets=256)
  tables = [_table("table_a", 64, 12, quantization_config=q1),
            _table("table_b", 120, 10, quantization_config=q2),
            _table("table_c", 120, 10, quantization_config=None)]
  features = [_feature(f"feature_spec_{n}", t)
              for n, t in zip("abc", tables)]
  table_stacking.auto_stack_tables(features, global_device_count=1,
                                   num_sc_per_device=4)
  assert [f.table_spec.setting_in_stack.stack_name for f in features] == [
      "table_a", "table_b", "table_c"]
  assert features[0].table_spec.stacked_table_spec.quantization_config == q1
  assert features[1].table_spec.stacked_table_spec.quantization_config == q2
  assert features[2].table_spec.stacked_table_spec.quantization_config is None


def test_manual_stacking_different_quantization_configs_raises():
  q1 = embedding_spec.QuantizationConfig(min_value=-5.0, max_value=5.0,
                                         num_buckets=256)
  q2 = embedding_spec.QuantizationConfig(min_value=-2.0, max_value=2.0,
                                         num_buckets=256)
  features = [_feature("feature_spec_a",
                       _table("table_a", 64, 12, quantization_config=q1)),
              _feature("feature_spec_b",
                       _table("table_b", 120, 10, quantization_config=q2))]
  with pytest.raises(ValueError, match="different quantization configs"):
    table_stacking.stack_tables(features, ["table_a", "table_b"],
                                global_device_count=1, num_sc_per_device=4)


# --- embedding_test.py ------------------------------------------------------


@pytest.mark.parametrize("num_sc,devices", SG)
def test_prepare_features_for_training_with_feature_stacking(num_sc, devices):
  table = embedding_spec.TableSpec(
      vocabulary_size=32, embedding_dim=12, initializer=None,
      optimizer=embedding_spec.SGDOptimizerSpec(), combiner="sum",
      name="table")
  fa = embedding_spec.FeatureSpec(table_spec=table, input_shape=[16, 1],
                                  output_shape=[16, 16], name="feature_a")
  fb = embedding_spec.FeatureSpec(table_spec=table, input_shape=[16, 1],
                                  output_shape=[16, 16], name="feature_b")
  embedding.prepare_feature_specs_for_training(
      (fa, fb), global_device_count=devices, num_sc_per_device=num_sc)
  expected = embedding_spec.StackedTableSpec(
      stack_name="table",
      stack_vocab_size=_round_up(32, 8 * devices * num_sc),
      stack_embedding_dim=16, combiner="sum",
      optimizer=embedding_spec.SGDOptimizerSpec(),
      max_ids_per_partition=256, max_unique_ids_per_partition=256,
      total_sample_count=32)
  assert fa.table_spec.setting_in_stack.stack_name == "table"
  assert fb.table_spec.setting_in_stack.stack_name == "table"
  assert fa.table_spec.stacked_table_spec == expected
  assert fb.table_spec.stacked_table_spec == expected
  assert fa.id_transformation.row_offset == 0
  assert fb.id_transformation.row_offset == 16


def _manual_settings_specs(stacked: bool):
  stack = embedding_spec.StackedTableSpec(
      stack_name="table_a_table_b", stack_vocab_size=74,
      stack_embedding_dim=16, combiner="sum",
      optimizer=embedding_spec.SGDOptimizerSpec(), max_ids_per_partition=16,
      max_unique_ids_per_partition=16, total_sample_count=32)
  extra_a = {"_stacked_table_spec": stack} if stacked else {}
  extra_b = {"_stacked_table_spec": stack} if stacked else {}
  t1 = embedding_spec.TableSpec(
      vocabulary_size=32 if stacked else 256, embedding_dim=16,
      initializer=None, optimizer=embedding_spec.SGDOptimizerSpec(),
      combiner="sum", name="table_a", max_ids_per_partition=16,
      max_unique_ids_per_partition=16,
      _setting_in_stack=embedding_spec.TableSettingInStack(
          stack_name="table_a_table_b" if stacked else "table_a",
          padded_vocab_size=32, padded_embedding_dim=16,
          row_offset_in_shard=0, shard_rotation=1), **extra_a)
  t2 = embedding_spec.TableSpec(
      vocabulary_size=42, embedding_dim=8, initializer=None,
      optimizer=embedding_spec.SGDOptimizerSpec(), combiner="sum",
      name="table_b", max_ids_per_partition=16,
      max_unique_ids_per_partition=16,
      _setting_in_stack=embedding_spec.TableSettingInStack(
          stack_name="table_a_table_b" if stacked else "table_b",
          padded_vocab_size=42, padded_embedding_dim=16 if stacked else 10,
          row_offset_in_shard=8, shard_rotation=2), **extra_b)
  f1 = embedding_spec.FeatureSpec(
      table_spec=t1, input_shape=[16, 1], output_shape=[16, 16],
      name="feature_a",
      _id_transformation=embedding_spec.FeatureIdTransformation(
          row_offset=0, col_offset=0, col_shift=1))
  f2 = embedding_spec.FeatureSpec(
      table_spec=t2, input_shape=[16, 1], output_shape=[16, 16],
      name="feature_b",
      _id_transformation=embedding_spec.FeatureIdTransformation(
          row_offset=16, col_offset=8, col_shift=2))
  return [f1, f2], stack


def test_manual_stacking_settings_error():
  features, _ = _manual_settings_specs(stacked=False)
  with pytest.raises(
      ValueError,
      match="embedding.prepare_feature_specs_for_training was not called"):
    embedding.get_stacked_table_specs(tuple(features))


@pytest.mark.parametrize("num_sc", [1, 2, 4])
def test_manual_stacking_settings(num_sc):
  features, stack = _manual_settings_specs(stacked=True)
  embedding.prepare_feature_specs_for_training(
      features, global_device_count=1, num_sc_per_device=num_sc)
  assert embedding.get_stacked_table_specs(features) == {
      "table_a_table_b": embedding_spec.StackedTableSpec(
          stack_name="table_a_table_b", stack_vocab_size=74,
          stack_embedding_dim=16, combiner="sum",
          optimizer=embedding_spec.SGDOptimizerSpec(),
          max_ids_per_partition=16, max_unique_ids_per_partition=16,
          total_sample_count=32)}
  assert features[0].table_spec.stacked_table_spec == stack
  # Settings given by hand are kept as they are.
  assert features[1].id_transformation == (
      embedding_spec.FeatureIdTransformation(row_offset=16, col_offset=8,
                                             col_shift=2))
  assert features[1].table_spec.setting_in_stack.shard_rotation == 2


# The reference's literals hold on the multi-device TPU slices it runs on:
# row_offset_in_shard 8 needs 32 / (8 * num_sparsecores) to round up to one
# row per shard (4+ SparseCores), shard_rotation = num_sc_per_device needs
# more SparseCores in total than per device (rotations are taken modulo the
# total).
@pytest.mark.parametrize("num_sc,devices", [(2, 2), (1, 4), (4, 2), (2, 4),
                                            (4, 4)])
def test_create_proto_from_feature_specs(num_sc, devices):
  a = embedding_spec.TableSpec(vocabulary_size=32, embedding_dim=14,
                               initializer=None, name="table_a")
  b = embedding_spec.TableSpec(vocabulary_size=128, embedding_dim=14,
                               initializer=None, name="table_b")
  features = [
      embedding_spec.FeatureSpec(table_spec=a, input_shape=[16, 1],
                                 output_shape=[16, 14], name="feature_a"),
      embedding_spec.FeatureSpec(table_spec=b, input_shape=[16, 1],
                                 output_shape=[16, 14], name="feature_b")]
  embedding.auto_stack_tables(features, num_sc_per_device=num_sc,
                              global_device_count=devices,
                              activation_mem_bytes_limit=64 * 1024 * 1024)
  ns = num_sc * devices
  pa, pb = _round_up(32, 8 * ns), _round_up(128, 8 * ns)
  expected = embedding_spec_pb2.EmbeddingSpecProto()
  text_format.Parse(f"""stacked_table_specs {{
      stack_name: "table_a_table_b"
      stack_vocab_size: {pa + pb}
      stack_embedding_dim: 16
      total_sample_count: 32
      max_ids_per_partition: 256
      max_unique_ids_per_partition: 256
      num_sparsecores: {ns}
      activation_mem_bytes_limit: 67108864
      table_specs {{
        table_name: "table_a"
        vocab_size: 32
        embedding_dim: 14
        padded_vocab_size: {pa}
        padded_embedding_dim: 16
        row_offset_in_shard: 0
        shard_rotation: 0
        feature_specs {{
          feature_name: "feature_a"
          input_shape: 16
          input_shape: 1
          output_shape: 16
          output_shape: 14
          row_offset: 0
          col_offset: 0
          col_shift: 0
        }}
        combiner: "sum"
        optimizer {{
          type: SGD
          learning_rate: 0.001
        }}
      }}
      table_specs {{
        table_name: "table_b"
        vocab_size: 128
        embedding_dim: 14
        padded_vocab_size: {pb}
        padded_embedding_dim: 16
        row_offset_in_shard: 8
        shard_rotation: {num_sc}
        feature_specs {{
          feature_name: "feature_b"
          input_shape: 16
          input_shape: 1
          output_shape: 16
          output_shape: 14
          row_offset: 16
          col_offset: {pa}
          col_shift: {num_sc}
        }}
        combiner: "sum"
        optimizer {{
          type: SGD
          learning_rate: 0.001
        }}
      }}
    }}""", expected)
  actual = embedding.create_proto_from_feature_specs(
      features, global_device_count=devices, num_sparsecore_per_device=num_sc)
  assert text_format.MessageToString(actual) == text_format.MessageToString(
      expected)
  assert actual.stacked_table_specs[0].activation_mem_bytes_limit == 67108864
  # The wire format round-trips.
  assert embedding_spec_pb2.EmbeddingSpecProto.FromString(
      actual.SerializeToString()) == actual


# Proto floats are float32: the parameters are chosen exactly representable.
@pytest.mark.parametrize("opt", [
    embedding_spec.SGDOptimizerSpec(learning_rate=0.25),
    embedding_spec.AdagradOptimizerSpec(learning_rate=0.5,
                                        initial_accumulator_value=0.25),
    embedding_spec.AdamOptimizerSpec(learning_rate=0.5, beta_1=0.75,
                                     beta_2=0.875, epsilon=2.0**-20),
    embedding_spec.FTRLOptimizerSpec(
        learning_rate=0.5, learning_rate_power=-0.5,
        l1_regularization_strength=0.125, l2_regularization_strength=0.25,
        beta=0.5, initial_accumulator_value=0.125,
        initial_linear_value=0.0, multiply_linear_by_learning_rate=True),
    embedding_spec.AdagradMomentumOptimizerSpec(
        learning_rate=0.5, momentum=0.75, beta2=1.0, epsilon=2.0**-10,
        exponent=2.0, use_nesterov=True, initial_accumulator_value=0.125,
        initial_momentum_value=0.0),
    embedding_spec.F2AOptimizerSpec(
        learning_rate=0.5, rho=0.25, initial_accumulator_value=0.125,
        initial_local_step_value=0.0, l1_regularization_strength=0.0625,
        l2_regularization_strength=0.03125, max_lr_multiplier=8.0),
])
def test_optimizer_proto_round_trip(opt):
  proto = embedding.optimizer_spec_to_proto(opt)
  assert embedding.proto_to_optimizer_spec(proto) == opt


def test_optimizer_proto_callable_learning_rate_and_laprop():
  def schedule(step):
    return 0.1 / (step + 1)

  proto = embedding.optimizer_spec_to_proto(
      embedding_spec.SGDOptimizerSpec(learning_rate=schedule))
  assert proto.WhichOneof("learning_rate_spec") == "learning_rate_tag"
  back = embedding.proto_to_optimizer_spec(proto)
  assert back.learning_rate == embedding_spec.CallablePlaceholder(
      proto.learning_rate_tag)
  with pytest.raises(RuntimeError, match="cannot be evaluated"):
    back.learning_rate(0)
  # LaProp has no value of its own in the schema.
  proto = embedding.optimizer_spec_to_proto(
      embedding_spec.LaPropOptimizerSpec())
  assert proto.type == embedding_spec_pb2.OptimizerSpecProto.CUSTOM
  assert isinstance(embedding.proto_to_optimizer_spec(None),
                    embedding_spec.SGDOptimizerSpec)
