"""Known-answer tests of the lookup and the fused updates, transcribed from
the reference's primitive tests (closed-form expectations that ran on TPU):

  forward   lib/core/primitives/tests/sparse_dense_matmul_csr_test.py:343-393
            (table row i holds i, one id per sample: activation = id) and
            :499-556 (1-D table id + 1, each sample holds its id twice:
            activation = 2 (id + 1))
  SGD       lib/core/primitives/tests/sparse_dense_matmul_grad_with_sgd_test.py:
            92-163 (grad 0.01, lr 0.01: touched rows - 1e-4, clipped to
            [2, 12] when clipping)
  Adagrad   lib/core/primitives/tests/sparse_dense_matmul_grad_with_adagrad_
            test.py:292-440 (row i holds i + 1, accumulator 0.002, grad
            0.012, lr 0.1: a = 0.002 + 0.012^2, row - 0.1 * 0.012 / sqrt(a),
            clipped when clipping; untouched rows unchanged)

Each case runs on the CPU oracle (CSR from oracle/refcpu.preprocess, lookup
and update from oracle/refcpu) and, marked gpu, on the product path (CSR from
lib/core/input_preprocessing on the GPU, primitives bound as in the reference
tests), for 1, 2 and 4 SparseCores per device. The reference compares with
assert_equal for the forward and atol 1e-5 for the updates; so do these.
"""

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore.lib.core import input_preprocessing
from jax_tpu_embedding.sparsecore.utils import utils
from oracle import refcpu

IDS = np.array([5, 3, 9, 1, 6, 12, 0, 4, 15, 13, 11, 7, 8, 14, 2, 10],
               np.int32).reshape(16, 1)
VOCAB, DIM, BATCH = 32, 8, 16


def _gpu():
  torch = pytest.importorskip("torch")
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  return torch


def _oracle_csr(ids, num_sc, max_ids=16):
  fs = input_preprocessing.single_feature_spec(
      ids.shape[0], int(ids.max()), max_ids, 64, 1, num_sc)
  r = refcpu.preprocess([ids], [np.ones_like(ids, np.float32)], [fs], 1, 1,
                        num_sc_per_device=num_sc)
  name = fs.table_spec.stacked_table_spec.stack_name
  return (r.row_pointers[name], r.embedding_ids[name], r.sample_ids[name],
          r.gains[name])


def _gpu_csr(ids, num_sc, max_ids=16):
  return input_preprocessing.preprocess_sparse_dense_matmul_input(
      ids, np.ones_like(ids, np.float32), 1, max_ids_per_partition=max_ids,
      max_unique_ids_per_partition=64, num_sc_per_device=num_sc)


def _shard(table, num_sc):
  return np.ascontiguousarray(
      utils.shard_emb_table(table, num_devices=1, num_sc_per_device=num_sc)[0])


def _unshard(table, num_sc):
  return utils.unshard_emb_table(np.asarray(table)[np.newaxis],
                                 num_sc_per_device=num_sc)


def _ids_table():
  return np.repeat(np.arange(VOCAB, dtype=np.float32)[:, None], DIM, axis=1)


def _expected_forward():
  return np.repeat(IDS.astype(np.float32), DIM, axis=1)


def _dim1_input():
  two = np.concatenate([IDS, IDS], axis=1)
  return np.concatenate([two, two], axis=0)


def _expected_dim1():
  single = (IDS[:, 0].astype(np.float32) + 1.0) * 2.0
  return np.concatenate([single, single])


def _expected_sgd(lo, hi):
  exp = _ids_table()
  rows = np.unique(IDS)
  exp[rows] -= 1e-4
  exp[rows] = np.clip(exp[rows], lo, hi)
  return exp


def _expected_adagrad(lo, hi):
  table = _ids_table() + 1.0
  acc = np.full(table.shape, 0.002, np.float64)
  rows = np.unique(IDS)
  a = 0.002 + 0.012 * 0.012
  exp_t = table.astype(np.float64)
  exp_t[rows] = np.clip(exp_t[rows] - 0.1 * 0.012 / np.sqrt(a), lo, hi)
  exp_a = acc.copy()
  exp_a[rows] = a
  return table, exp_t, exp_a


CLIPS = [(None, None), (2.0, 12.0)]


@pytest.mark.parametrize("num_sc", [1, 2, 4])
def test_oracle_forward_kats(num_sc):
  csr = _oracle_csr(IDS, num_sc)
  act = refcpu.sparse_dense_matmul(*csr, _shard(_ids_table(), num_sc), BATCH,
                                   num_sc_per_device=num_sc, num_scs=num_sc)
  np.testing.assert_equal(act, _expected_forward())
  # 32 deduplicated ids: with one SparseCore they share one partition.
  csr = _oracle_csr(_dim1_input(), num_sc, max_ids=32)
  table = _shard(np.arange(VOCAB, dtype=np.float32) + 1.0, num_sc)
  act = refcpu.sparse_dense_matmul(*csr, table, 2 * BATCH,
                                   num_sc_per_device=num_sc, num_scs=num_sc)
  np.testing.assert_allclose(act, _expected_dim1(), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("lo,hi", CLIPS)
def test_oracle_sgd_kat(num_sc, lo, hi):
  csr = _oracle_csr(IDS, num_sc)
  grad = np.full((BATCH, DIM), 0.01, np.float32)
  got = refcpu.sparse_dense_matmul_grad(
      *csr, grad, _shard(_ids_table(), num_sc), None, learning_rate=0.01,
      num_sc_per_device=num_sc, num_scs=num_sc, min_value=lo, max_value=hi)
  np.testing.assert_allclose(_unshard(got, num_sc), _expected_sgd(lo, hi),
                             atol=1e-5)


@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("lo,hi", CLIPS)
def test_oracle_adagrad_kat(num_sc, lo, hi):
  csr = _oracle_csr(IDS, num_sc)
  table, exp_t, exp_a = _expected_adagrad(lo, hi)
  grad = np.full((BATCH, DIM), 0.012, np.float32)
  acc = np.full(table.shape, 0.002, np.float32)
  got_t, got_a = refcpu.sparse_dense_matmul_grad(
      *csr, grad, _shard(table, num_sc), _shard(acc, num_sc),
      learning_rate=0.1, num_sc_per_device=num_sc, num_scs=num_sc,
      min_value=lo, max_value=hi)
  np.testing.assert_allclose(_unshard(got_a, num_sc), exp_a, atol=1e-5)
  np.testing.assert_allclose(_unshard(got_t, num_sc), exp_t, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("num_sc", [1, 2, 4])
def test_gpu_forward_kats(num_sc):
  torch = _gpu()
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr  # pylint: disable=g-import-not-at-top

  bind = sparse_dense_matmul_csr.tpu_sparse_dense_matmul_csr_primitive.bind
  kw = dict(max_ids_per_partition=16, max_unique_ids_per_partition=16,
            sharding_strategy=1, quantization_config=None,
            enable_minibatching=False, num_sc_per_device=num_sc)
  csr = _gpu_csr(IDS, num_sc)
  act = bind(*csr, 1, torch.from_numpy(_shard(_ids_table(), num_sc)).cuda(),
             device_batch_size=BATCH, **kw)
  np.testing.assert_equal(act.cpu().numpy(), _expected_forward())
  csr = _gpu_csr(_dim1_input(), num_sc, max_ids=32)
  table = _shard(np.arange(VOCAB, dtype=np.float32) + 1.0, num_sc)
  act = bind(*csr, 1, torch.from_numpy(table).cuda(),
             device_batch_size=2 * BATCH, **kw)
  np.testing.assert_allclose(act.cpu().numpy(), _expected_dim1(), rtol=1e-5,
                             atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("lo,hi", CLIPS)
def test_gpu_sgd_kat(num_sc, lo, hi):
  torch = _gpu()
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd as sgd  # pylint: disable=g-import-not-at-top

  csr = _gpu_csr(IDS, num_sc)
  table = torch.from_numpy(_shard(_ids_table(), num_sc)).cuda()
  grad = torch.full((BATCH, DIM), 0.01, dtype=torch.float32, device="cuda")
  out = sgd.tpu_sparse_dense_matmul_grad_with_sgd_primitive.bind(
      *csr, 1, table, grad, 0.01, max_ids_per_partition=16,
      max_unique_ids_per_partition=16,
      computation_name="sgd_test_computation", sharding_strategy=1,
      min_value=lo, max_value=hi, num_sc_per_device=num_sc)
  np.testing.assert_allclose(_unshard(out.cpu().numpy(), num_sc),
                             _expected_sgd(lo, hi), atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("num_sc", [1, 2, 4])
@pytest.mark.parametrize("lo,hi", CLIPS)
def test_gpu_adagrad_kat(num_sc, lo, hi):
  torch = _gpu()
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as ada  # pylint: disable=g-import-not-at-top

  csr = _gpu_csr(IDS, num_sc)
  table, exp_t, exp_a = _expected_adagrad(lo, hi)
  acc = np.full(table.shape, 0.002, np.float32)
  got_t, got_a = ada.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
      *csr, 1, torch.from_numpy(_shard(table, num_sc)).cuda(),
      torch.from_numpy(_shard(acc, num_sc)).cuda(),
      torch.full((BATCH, DIM), 0.012, dtype=torch.float32, device="cuda"),
      np.float32(0.1), max_ids_per_partition=16,
      max_unique_ids_per_partition=16,
      computation_name="optimizer_test_computation", sharding_strategy=1,
      min_value=lo, max_value=hi, num_sc_per_device=num_sc)
  np.testing.assert_allclose(_unshard(got_a.cpu().numpy(), num_sc), exp_a,
                             atol=1e-5)
  np.testing.assert_allclose(_unshard(got_t.cpu().numpy(), num_sc), exp_t,
                             atol=1e-5)


def test_max_ids_must_be_positive():
  """Argument check of reference input_preprocessing.py:329-332."""
  with pytest.raises(ValueError, match="must be positive"):
    input_preprocessing.preprocess_sparse_dense_matmul_input(
        IDS, np.ones_like(IDS, np.float32), 1, max_ids_per_partition=0,
        max_unique_ids_per_partition=64)


@pytest.mark.gpu
def test_gpu_limits_raise_value_error_like_the_reference():
  """_validate_partition_map (reference input_preprocessing.py:96-122):
  sixteen samples of id 0 put 16 ids into one partition."""
  _gpu()
  with pytest.raises(ValueError, match="too many ids. 16 > 4"):
    input_preprocessing.preprocess_sparse_dense_matmul_input(
        np.zeros((16, 1), np.int32), np.ones((16, 1), np.float32), 1,
        max_ids_per_partition=4, max_unique_ids_per_partition=64,
        num_sc_per_device=1)
