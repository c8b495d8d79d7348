"""Full-buffer known-answer tests of preprocessing through the public API.

The expectations in tests/golden/pybind_kats.json are transcribed from the
reference's pybind_input_preprocessing_test.py. Each case runs on the CPU
oracle (always) and on the GPU path (marked gpu), and both must reproduce the
reference's buffers on the compared region and its stats exactly.
"""

import json
import os

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore.lib.nn import embedding
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from oracle import refcpu

_KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                    "pybind_kats.json")))
INT_MAX = 2**31 - 1


def _single_table_case(case):
  table = embedding_spec.TableSpec(
      name="table", vocabulary_size=case["vocab"], embedding_dim=case["dim"],
      optimizer=embedding_spec.SGDOptimizerSpec(0.001), combiner="sum",
      max_ids_per_partition=case["max_ids"],
      max_unique_ids_per_partition=case["max_ids"])
  feats = np.array(case["features"], np.int32)
  fs = embedding_spec.FeatureSpec(name="feature", table_spec=table,
                                  input_shape=list(feats.shape),
                                  output_shape=[feats.shape[0], case["dim"]])
  embedding.prepare_feature_specs_for_training(
      fs, global_device_count=case["global_device_count"],
      num_sc_per_device=case["num_sc_per_device"])
  weights = np.ones_like(feats, dtype=np.float32)
  return [feats], [weights], [fs]


def _expected(case, key, fill):
  out = np.full(case["coo_size"], fill,
                np.float32 if key == "gains" else np.int32)
  for pos, v in case[key]:
    out[pos] = v
  return out


def _assert_region(rp, got, exp, segments):
  for rp_s, g_s, e_s in zip(np.split(rp, segments), np.split(got, segments),
                            np.split(exp, segments)):
    n = int(rp_s[-1])
    np.testing.assert_array_equal(g_s[:n], e_s[:n])


def _check(case, rp, eid, sid, gains):
  s = case["num_sc_per_device"]
  np.testing.assert_array_equal(rp, np.array(case["row_pointers"], np.int32))
  _assert_region(rp, eid, _expected(case, "embedding_ids", INT_MAX), s)
  _assert_region(rp, sid, _expected(case, "sample_ids", INT_MAX), s)
  _assert_region(rp, gains, _expected(case, "gains", np.nan), s)


def _fdo_specs(case):
  opt = embedding_spec.SGDOptimizerSpec(0.001)
  stacked = embedding_spec.StackedTableSpec(
      stack_name="one_table_to_rule_them_all",
      stack_vocab_size=case["stack_vocab"], stack_embedding_dim=8,
      optimizer=opt, combiner="sum", total_sample_count=16,
      max_ids_per_partition=case["max_ids"],
      max_unique_ids_per_partition=case["max_ids"])
  specs = []
  for name, vocab, shape, ro, co in (("a", 32, [16, 8], 0, 0),
                                     ("b", 16, [16, 4], 8, 32)):
    t = embedding_spec.TableSpec(
        name=f"table_{name}", vocabulary_size=vocab, embedding_dim=8,
        optimizer=opt, combiner="sum", max_ids_per_partition=8,
        max_unique_ids_per_partition=8,
        _setting_in_stack=embedding_spec.TableSettingInStack(
            stack_name="one_table_to_rule_them_all", padded_vocab_size=48,
            padded_embedding_dim=8),
        _stacked_table_spec=stacked)
    specs.append(embedding_spec.FeatureSpec(
        name=f"feature_spec_{name}", table_spec=t, input_shape=shape,
        output_shape=[shape[0] // 2, 8],
        _id_transformation=embedding_spec.FeatureIdTransformation(
            row_offset=ro, col_offset=co, col_shift=0)))
  feats = [np.array(case["features_a"], np.int32),
           np.array(case["features_b"], np.int32)]
  weights = [np.ones_like(f, dtype=np.float32) for f in feats]
  return feats, weights, specs


@pytest.mark.parametrize("name", ["single_column", "multiple_columns"])
def test_oracle_full_buffers(name):
  case = _KATS[name]
  feats, weights, specs = _single_table_case(case)
  r = refcpu.preprocess(feats, weights, specs, 1, case["global_device_count"],
                        num_sc_per_device=case["num_sc_per_device"])
  _check(case, r.row_pointers["table"], r.embedding_ids["table"],
         r.sample_ids["table"], r.gains["table"])


def test_oracle_multi_process_stats():
  case = _KATS["multi_process_fdo"]
  feats, weights, specs = _fdo_specs(case)
  r = refcpu.preprocess(feats, weights, specs, case["local_device_count"],
                        case["global_device_count"],
                        num_sc_per_device=case["num_sc_per_device"])
  name = "one_table_to_rule_them_all"
  np.testing.assert_array_equal(r.max_ids_per_partition[name],
                                case["max_ids_per_partition"])
  np.testing.assert_array_equal(r.max_unique_ids_per_partition[name],
                                case["max_unique_ids_per_partition"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["single_column", "multiple_columns"])
@pytest.mark.parametrize("unity", [False, True])
def test_gpu_full_buffers(name, unity):
  torch = pytest.importorskip("torch")
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  case = _KATS[name]
  feats, weights, specs = _single_table_case(case)
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      feats, None if unity else weights, specs, 1,
      case["global_device_count"], num_sc_per_device=case["num_sc_per_device"])
  _check(case, pre.lhs_row_pointers["table"].cpu().numpy(),
         pre.lhs_embedding_ids["table"].cpu().numpy(),
         pre.lhs_sample_ids["table"].cpu().numpy(),
         pre.lhs_gains["table"].cpu().numpy())


@pytest.mark.gpu
def test_gpu_multi_process_stats():
  torch = pytest.importorskip("torch")
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  case = _KATS["multi_process_fdo"]
  feats, weights, specs = _fdo_specs(case)
  _, stats = embedding.preprocess_sparse_dense_matmul_input(
      feats, weights, specs, case["local_device_count"],
      case["global_device_count"], num_sc_per_device=case["num_sc_per_device"])
  name = "one_table_to_rule_them_all"
  np.testing.assert_array_equal(stats.max_ids_per_partition[name],
                                case["max_ids_per_partition"])
  np.testing.assert_array_equal(stats.max_unique_ids_per_partition[name],
                                case["max_unique_ids_per_partition"])
