"""The batched host-to-device staging used by preprocessing
(_native.HostUploads): every array arrives intact, 256-byte aligned, in one
copy, whatever its dtype or size (empty included)."""

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore import _native


def _torch():
  torch = pytest.importorskip("torch")
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  return torch


@pytest.mark.gpu
def test_arrays_arrive_intact_and_aligned():
  torch = _torch()
  rng = np.random.default_rng(0)
  arrays = [
      (rng.integers(-2**31, 2**31 - 1, 1001).astype(np.int32), torch.int32),
      (np.zeros(0, np.int64), torch.int64),
      (rng.integers(0, 2**40, 17).astype(np.int64), torch.int64),
      (rng.standard_normal(3).astype(np.float32), torch.float32),
      (np.arange(5, dtype=np.int64), torch.int32),  # converted on the host
      (np.zeros(0, np.float32), torch.float32),
  ]
  up = _native.HostUploads()
  handles = [up.add(a, dt) for a, dt in arrays]
  with pytest.raises(RuntimeError, match="flush"):
    _native.HostUploads.resolve(handles[0])
  up.flush()
  for (a, dt), h in zip(arrays, handles):
    got = _native.HostUploads.resolve(h)
    assert got.is_cuda and got.dtype == dt and got.numel() == a.size
    assert got.data_ptr() % 256 == 0
    np.testing.assert_array_equal(got.cpu().numpy(),
                                  a.astype(got.cpu().numpy().dtype))
  # Anything that is not a handle resolves to itself.
  assert _native.HostUploads.resolve(None) is None
  # A second batch on the same stager starts afresh.
  h = up.add(np.array([7, 8, 9], np.int32), torch.int32)
  up.flush()
  np.testing.assert_array_equal(_native.HostUploads.resolve(h).cpu().numpy(),
                                [7, 8, 9])


@pytest.mark.gpu
def test_row_splits_checked_while_staged():
  """Row splits are checked in the same pass that stages them: valid ones
  arrive intact with their longest row; invalid ones raise ValueError from
  flush(), as does preprocessing a feature that holds them."""
  torch = _torch()
  up = _native.HostUploads()
  ids = up.add(np.arange(9, dtype=np.int32), torch.int32)
  good = up.add_row_splits(np.array([0, 2, 2, 7, 9], np.int64), 9)
  up.flush()
  np.testing.assert_array_equal(
      _native.HostUploads.resolve(good).cpu().numpy(), [0, 2, 2, 7, 9])
  assert good.max_row_length == 5
  np.testing.assert_array_equal(
      _native.HostUploads.resolve(ids).cpu().numpy(), np.arange(9))
  up = _native.HostUploads()
  up.add_row_splits(np.array([0, 4, 3, 9], np.int64), 9)
  with pytest.raises(ValueError, match="non-decreasing"):
    up.flush()
  with pytest.raises(ValueError, match="non-decreasing"):
    up.add_row_splits(np.zeros(0, np.int64), 0)

  from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top
  t = embedding_spec.TableSpec(
      name="t", vocabulary_size=16, embedding_dim=8,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner="sum",
      max_ids_per_partition=64, max_unique_ids_per_partition=64)
  fs = embedding_spec.FeatureSpec(name="f", table_spec=t, input_shape=[4, 1],
                                  output_shape=[4, 8])
  embedding.prepare_feature_specs_for_training([fs], 1, 1)
  bad = pip.RaggedIds(np.arange(6, dtype=np.int32),
                      np.array([0, 3, 2, 5, 6], np.int64))
  with pytest.raises(ValueError, match="non-decreasing"):
    pip.preprocess_sparse_dense_matmul_input([bad], None, [fs], 1, 1,
                                             num_sc_per_device=1)
