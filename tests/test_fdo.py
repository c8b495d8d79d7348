"""FDO clients: record / publish / load of preprocessing stats, transcribed
from the reference's tests (lib/fdo/file_fdo_client_test.py:24-152,
lib/fdo/csv_file_fdo_client_test.py:26-181), plus the round trip into
update_preprocessing_parameters and two processes sharing one store."""

import csv

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore.lib.fdo import csv_file_fdo_client
from jax_tpu_embedding.sparsecore.lib.fdo import fdo_client
from jax_tpu_embedding.sparsecore.lib.fdo import file_fdo_client
from jax_tpu_embedding.sparsecore.lib.nn import embedding
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec

CLIENTS = {
    "npz": file_fdo_client.NPZFileFDOClient,
    "csv": csv_file_fdo_client.CSVFileFDOClient,
}


def _assert_stats_equal(actual, expected):
  assert len(actual) == len(expected)
  for key in expected:
    assert key in actual
    np.testing.assert_array_equal(expected[key], actual[key])


def _stats(max_ids, max_unique, buf):
  return embedding.SparseDenseMatmulInputStats(
      max_ids_per_partition=max_ids, max_unique_ids_per_partition=max_unique,
      required_buffer_size_per_sc=buf)


@pytest.mark.parametrize("kind", sorted(CLIENTS))
def test_record_and_publish_load(kind, tmp_path):
  client = CLIENTS[kind](tmp_path)
  stats = _stats({"tab_one": np.array([10, 20, 30, 40])},
                 {"tab_one": np.array([1, 2, 3, 4])}, {})
  client.record(stats)
  client.publish()
  loaded = client.load()
  _assert_stats_equal(loaded.max_ids_per_partition,
                      stats.max_ids_per_partition)
  _assert_stats_equal(loaded.max_unique_ids_per_partition,
                      stats.max_unique_ids_per_partition)
  _assert_stats_equal(loaded.required_buffer_size_per_sc, {})


@pytest.mark.parametrize("kind", sorted(CLIENTS))
def test_multiple_record_keeps_history(kind, tmp_path):
  client = CLIENTS[kind](tmp_path)
  stats = _stats({"tab_one": np.array([10, 20, 30, 40])},
                 {"tab_one": np.array([1, 2, 3, 4])},
                 {"tab_one": np.array([256])})
  client.record(stats)
  client.record(stats)
  client.publish()
  loaded = client.load()
  _assert_stats_equal(
      loaded.max_ids_per_partition,
      {"tab_one": np.array([[10, 20, 30, 40], [10, 20, 30, 40]])})
  _assert_stats_equal(
      loaded.max_unique_ids_per_partition,
      {"tab_one": np.array([[1, 2, 3, 4], [1, 2, 3, 4]])})
  _assert_stats_equal(loaded.required_buffer_size_per_sc,
                      {"tab_one": np.array([[256], [256]])})


def test_csv_without_history_keeps_the_maximum(tmp_path):
  client = csv_file_fdo_client.CSVFileFDOClient(tmp_path,
                                                retain_history=False)
  client.record(_stats({"tab_one": np.array([10, 20, 30, 40])},
                       {"tab_one": np.array([1, 2, 3, 4])},
                       {"tab_one": np.array([256])}))
  client.record(_stats({"tab_one": np.array([5, 25, 15, 45])},
                       {"tab_one": np.array([0, 3, 2, 5])},
                       {"tab_one": np.array([512])}))
  client.publish()
  loaded = client.load()
  _assert_stats_equal(loaded.max_ids_per_partition,
                      {"tab_one": np.array([10, 25, 30, 45])})
  _assert_stats_equal(loaded.max_unique_ids_per_partition,
                      {"tab_one": np.array([1, 3, 3, 5])})
  _assert_stats_equal(loaded.required_buffer_size_per_sc,
                      {"tab_one": np.array([512])})


_FILE_0 = {
    "t_one_max_ids": [10, 20, 30, 40], "t_two_max_ids": [50, 60, 70, 80],
    "t_one_max_unique_ids": [1, 2, 3, 4], "t_two_max_unique_ids": [5, 6, 7, 8],
    "t_one_required_buffer_size": [64], "t_two_required_buffer_size": [128],
}
_FILE_1 = {
    "t_one_max_ids": [20, 10, 40, 30], "t_two_max_ids": [60, 60, 80, 70],
    "t_one_max_unique_ids": [2, 1, 4, 3], "t_two_max_unique_ids": [6, 5, 8, 7],
    "t_one_required_buffer_size": [128], "t_two_required_buffer_size": [256],
}


def _write_files(kind, base):
  for name, content in (("fdo_stats_0_10", _FILE_0),
                        ("fdo_stats_1_11", _FILE_1)):
    if kind == "npz":
      np.savez(base / f"{name}.npz",
               **{k: np.array(v) for k, v in content.items()})
    else:
      with open(base / f"{name}.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["key", "values"])
        for k, v in content.items():
          w.writerow([k, " ".join(map(str, v))])


@pytest.mark.parametrize("kind", sorted(CLIENTS))
def test_load_takes_the_maximum_over_processes(kind, tmp_path):
  _write_files(kind, tmp_path)
  loaded = CLIENTS[kind](tmp_path).load()
  _assert_stats_equal(loaded.max_ids_per_partition,
                      {"t_one": np.array([20, 20, 40, 40]),
                       "t_two": np.array([60, 60, 80, 80])})
  _assert_stats_equal(loaded.max_unique_ids_per_partition,
                      {"t_one": np.array([2, 2, 4, 4]),
                       "t_two": np.array([6, 6, 8, 8])})
  _assert_stats_equal(loaded.required_buffer_size_per_sc,
                      {"t_one": np.array([128]), "t_two": np.array([256])})


@pytest.mark.parametrize("kind", sorted(CLIENTS))
def test_files_not_found(kind, tmp_path):
  with pytest.raises(FileNotFoundError):
    CLIENTS[kind](tmp_path).load()


def test_unexpected_key_raises(tmp_path):
  np.savez(tmp_path / "fdo_stats_0_1.npz", t_one_bogus=np.array([1]))
  with pytest.raises(ValueError, match="Unexpected key"):
    file_fdo_client.NPZFileFDOClient(tmp_path).load()


def test_latest_files_by_process(tmp_path):
  files = [
      "temp/fdo_dumps/fdo_stats_0_10.npz",
      "temp/fdo_dumps/fdo_stats_0_20.npz",
      "temp/fdo_dumps/fdo_stats_0_30.npz",
      "temp/fdo_dumps/fdo_stats_1_09.npz",
      "temp/fdo_dumps/fdo_stats_0_40.npz",
      "temp/fdo_dumps/fdo_stats_2_10.npz",
  ]
  client = file_fdo_client.NPZFileFDOClient(tmp_path)
  assert client._get_latest_files_by_process(files) == [  # pylint: disable=protected-access
      "temp/fdo_dumps/fdo_stats_2_10.npz",
      "temp/fdo_dumps/fdo_stats_1_09.npz",
      "temp/fdo_dumps/fdo_stats_0_40.npz",
  ]


@pytest.mark.parametrize("kind", sorted(CLIENTS))
def test_two_processes_share_a_store(kind, tmp_path, monkeypatch):
  """Each process publishes its own file; load() on either sees the
  element-wise maximum, and the newer file of a process replaces its older
  one. Drop counters (scalars) survive the round trip."""
  for rank, (ids, drops) in enumerate(((np.array([3, 9]), 0),
                                       (np.array([7, 2]), 5))):
    monkeypatch.setattr(fdo_client, "process_index", lambda r=rank: r)
    c = CLIENTS[kind](tmp_path)
    c.record(embedding.SparseDenseMatmulInputStats(
        max_ids_per_partition={"s": ids},
        max_unique_ids_per_partition={"s": ids // 2},
        required_buffer_size_per_sc={"s": np.array([16])},
        id_drop_counters={"s": drops}))
    c.publish()
  loaded = CLIENTS[kind](tmp_path).load()
  np.testing.assert_array_equal(loaded.max_ids_per_partition["s"], [7, 9])
  np.testing.assert_array_equal(loaded.max_unique_ids_per_partition["s"],
                                [3, 4])
  assert int(np.max(loaded.id_drop_counters["s"])) == 5
  # A newer file of process 1 with smaller stats replaces its older one.
  monkeypatch.setattr(fdo_client, "process_index", lambda: 1)
  c = CLIENTS[kind](tmp_path)
  c.record(_stats({"s": np.array([1, 1])}, {"s": np.array([1, 1])},
                  {"s": np.array([8])}))
  c.publish()
  loaded = CLIENTS[kind](tmp_path).load()
  np.testing.assert_array_equal(loaded.max_ids_per_partition["s"], [3, 9])


def test_round_trip_into_update_preprocessing_parameters(tmp_path):
  """Loaded stats become the stack limits and the buffer size
  (embedding.update_preprocessing_parameters)."""
  table = embedding_spec.TableSpec(
      name="t", vocabulary_size=64, embedding_dim=8,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner="sum",
      max_ids_per_partition=4, max_unique_ids_per_partition=4)
  fs = embedding_spec.FeatureSpec(name="f", table_spec=table,
                                  input_shape=[32, 1], output_shape=[32, 8])
  embedding.prepare_feature_specs_for_training([fs], 1, 4)
  name = fs.table_spec.stacked_table_spec.stack_name
  client = file_fdo_client.NPZFileFDOClient(tmp_path)
  client.record(_stats({name: np.array([5, 11, 2, 7])},
                       {name: np.array([5, 9, 2, 7])},
                       {name: np.array([32, 40, 16, 24])}))
  client.publish()
  loaded = client.load()
  embedding.update_preprocessing_parameters([fs], loaded, 4)
  st = fs.table_spec.stacked_table_spec
  assert st.max_ids_per_partition == 11
  assert st.max_unique_ids_per_partition == 9
  assert st.suggested_coo_buffer_size_per_device == 160
