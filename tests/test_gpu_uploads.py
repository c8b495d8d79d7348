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
