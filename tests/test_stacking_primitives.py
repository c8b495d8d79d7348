"""The activation-unstacking and gradient-stacking primitives.

Transcribed from the reference (paths under jax_tpu_embedding/sparsecore/):
  lib/core/primitives/tests/sparse_dense_matmul_activation_unstack_test.py:
      47-61 (abstract eval: two features of (128, 32) and (256, 64) from a
      (384, 64) stacked matrix), 63-104 (functional: an arange matrix, the
      features' row ranges and leading columns in sequence);
  lib/core/primitives/tests/sparse_dense_matmul_gradient_stack_test.py:
      46-61 (abstract eval: (128, 32) and (256, 32) into (384, 32)), 63-87
      (functional: ones and twos concatenated).
The reference mocks the implementations in those functional tests (its
custom calls run only on a TPU); here they run the HIP copies, so the mock's
expectation is the expectation. Beyond them, on the GPU: several
SparseCores (the interleaved layout, checked against the per-feature slices
the default unstacking takes, embedding.py:903-956), dims that are not
multiples of four (the 4-byte path), more than 32 row blocks (several
launches), stacked rows past the features and padding columns written as
zeros, and unstack(stack(g)) == g.
"""

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_activation_unstack as unstack_mod
from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_gradient_stack as stack_mod

UNSTACK = unstack_mod.tpu_sparse_dense_matmul_activation_unstack_primitive
STACK = stack_mod.tpu_sparse_dense_matmul_gradient_stack_primitive


def test_activation_unstack_abstract_eval():
  out = UNSTACK.abstract_eval(np.zeros((384, 64), np.float32),
                              per_feature_batch_sizes=(128, 256),
                              per_feature_dims=(32, 64))
  assert len(out) == 2
  assert out[0].shape == (128, 32) and out[0].dtype == np.float32
  assert out[1].shape == (256, 64) and out[1].dtype == np.float32
  assert UNSTACK.multiple_results


def test_gradient_stack_abstract_eval():
  g1 = np.zeros((128, 32), np.float32)
  g2 = np.zeros((256, 32), np.float32)
  out = STACK.abstract_eval(g1, g2, stacked_batch_size=384,
                            stacked_feature_dim=32)
  assert out.shape == (384, 32) and out.dtype == np.float32
  assert not STACK.multiple_results


torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def _gpu():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  torch.cuda.set_device(0)


@pytest.mark.gpu
def test_activation_unstack_functional(_gpu):  # pylint: disable=redefined-outer-name,unused-argument
  rows, dim = 128 + 256, 64
  x = np.arange(rows * dim, dtype=np.float32).reshape(rows, dim)
  outs = UNSTACK.bind(torch.from_numpy(x).cuda(),
                      per_feature_batch_sizes=(128, 256),
                      per_feature_dims=(32, 64), num_sc_per_device=1)
  assert len(outs) == 2
  np.testing.assert_array_equal(outs[0].cpu().numpy(), x[0:128, :32])
  np.testing.assert_array_equal(outs[1].cpu().numpy(), x[128:384, :64])


@pytest.mark.gpu
def test_gradient_stack_functional(_gpu):  # pylint: disable=redefined-outer-name,unused-argument
  g1 = np.ones((128, 32), np.float32)
  g2 = np.ones((256, 32), np.float32) * 2
  out = STACK.bind(torch.from_numpy(g1).cuda(), torch.from_numpy(g2).cuda(),
                   stacked_batch_size=384, stacked_feature_dim=32,
                   num_sc_per_device=1)
  np.testing.assert_array_equal(out.cpu().numpy(),
                                np.concatenate([g1, g2], axis=0))


def _interleaved_rows(batches, num_sc, rows):
  """Stacked row of each feature's output rows: the per-SparseCore slices
  of the default unstacking (embedding.py:925-955 with G = 1)."""
  seg = rows // num_sc
  out, cum = [], 0
  for b in batches:
    per = b // num_sc
    out.append(np.concatenate([
        s * seg + cum // num_sc + np.arange(per) for s in range(num_sc)
    ]).astype(np.int64) if b else np.zeros(0, np.int64))
    cum += b
  return out


@pytest.mark.gpu
@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("dims,stacked_dim", [
    ((8, 16, 8), 16),        # 16-byte path
    ((5, 3, 6, 1), 6),       # 4-byte path (width and dim not multiples of 4)
    (tuple([4, 8] * 20), 8),  # 40 features: more than 32 blocks
])
def test_interleaved_round_trip(_gpu, num_sc, dims, stacked_dim):  # pylint: disable=redefined-outer-name,unused-argument
  rng = np.random.default_rng(7 * num_sc + len(dims))
  batches = [int(num_sc * rng.integers(0, 9)) for _ in dims]
  batches[0] = 8 * num_sc  # at least one non-empty feature
  pad_rows = 4 * num_sc    # stacked rows past every feature
  rows = sum(batches) + pad_rows
  x = rng.normal(size=(rows, stacked_dim)).astype(np.float32)
  outs = UNSTACK.bind(torch.from_numpy(x).cuda(),
                      per_feature_batch_sizes=tuple(batches),
                      per_feature_dims=dims, num_sc_per_device=num_sc)
  where = _interleaved_rows(batches, num_sc, rows)
  for o, r, d in zip(outs, where, dims):
    np.testing.assert_array_equal(o.cpu().numpy(), x[r, :d])
  # Stacked back: the same rows and columns, zeros elsewhere.
  back = STACK.bind(*outs, stacked_batch_size=rows,
                    stacked_feature_dim=stacked_dim,
                    num_sc_per_device=num_sc).cpu().numpy()
  want = np.zeros_like(x)
  for r, d in zip(where, dims):
    want[r, :d] = x[r, :d]
  np.testing.assert_array_equal(back, want)


@pytest.mark.gpu
def test_validation_errors(_gpu):  # pylint: disable=redefined-outer-name,unused-argument
  x = torch.zeros((16, 8), dtype=torch.float32, device="cuda")
  with pytest.raises(ValueError, match="more than the"):
    UNSTACK.bind(x, per_feature_batch_sizes=(8, 16), per_feature_dims=(8, 8),
                 num_sc_per_device=1)
  with pytest.raises(ValueError, match="outside the stacked dim"):
    UNSTACK.bind(x, per_feature_batch_sizes=(8,), per_feature_dims=(9,),
                 num_sc_per_device=1)
  with pytest.raises(ValueError, match="multiple of 2"):
    UNSTACK.bind(x, per_feature_batch_sizes=(3,), per_feature_dims=(8,),
                 num_sc_per_device=2)
  with pytest.raises(ValueError, match="more than the stacked dim"):
    STACK.bind(torch.zeros((4, 9), device="cuda"), stacked_batch_size=16,
               stacked_feature_dim=8, num_sc_per_device=1)
  with pytest.raises(ValueError, match="more than the 4 stacked rows"):
    STACK.bind(torch.zeros((8, 8), device="cuda"), stacked_batch_size=4,
               stacked_feature_dim=8, num_sc_per_device=1)
