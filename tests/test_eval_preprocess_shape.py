"""eval_preprocess_sparse_dense_matmul_input_shape (embedding.py:822-900 of
the reference): the CSR buffers' shapes and dtypes from the specs alone.

Checked on the CPU against the buffers the oracle's preprocessing returns
for the same specs: a c5-like structure (six stacks of different dims with
feature stacking, ragged rows) and a c3-like one (weighted, two stacks split
by combiner), at one, two and four SparseCores, two local devices, with and
without minibatching. The full-size configurations are checked against the
GPU preprocessing in tests/test_configs_gpu.py.
"""

import numpy as np
import pytest

from jax_tpu_embedding.sparsecore.lib.nn import embedding
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec
from jax_tpu_embedding.sparsecore.lib.nn import table_stacking
from oracle import refcpu


def _specs(kind, batch, num_sc, local):
  opt = embedding_spec.AdagradOptimizerSpec(learning_rate=0.01)
  rng = np.random.default_rng(len(kind) + num_sc)
  feats, data, weights = [], [], []
  if kind == "c5":
    dims = [8, 16, 32, 64, 128, 256]
    tables = [embedding_spec.TableSpec(
        name=f"t{t:02d}", vocabulary_size=int(rng.integers(500, 5000)),
        embedding_dim=dims[t % 6], initializer=None, optimizer=opt,
        combiner="mean", max_ids_per_partition=1,
        max_unique_ids_per_partition=1) for t in range(12)]
    for f in range(14):
      t = tables[f % 12]
      feats.append(embedding_spec.FeatureSpec(
          name=f"f{f:02d}", table_spec=t, input_shape=[batch, 1],
          output_shape=[batch, t.embedding_dim]))
    groups = [([f for f in range(14) if f % 12 in (d, d + 6)],
               [f"t{d:02d}", f"t{d + 6:02d}"], f"s{d}") for d in range(6)]
  else:
    tables = [embedding_spec.TableSpec(
        name=f"t{t}", vocabulary_size=3000, embedding_dim=64,
        initializer=None, optimizer=opt,
        combiner="sqrtn" if t < 2 else "mean", max_ids_per_partition=1,
        max_unique_ids_per_partition=1) for t in range(4)]
    feats = [embedding_spec.FeatureSpec(
        name=f"f{t}", table_spec=tables[t], input_shape=[batch, 1],
        output_shape=[batch, 64]) for t in range(4)]
    groups = [([0, 1], ["t0", "t1"], "sqrtn"), ([2, 3], ["t2", "t3"], "mean")]
  for fs in feats:
    lens = rng.integers(1, 12, size=batch)
    v = fs.table_spec.vocabulary_size
    data.append(np.array([rng.integers(0, v, size=n).astype(np.int32)
                          for n in lens], dtype=object))
    weights.append(np.array([rng.uniform(0.1, 1, size=n).astype(np.float32)
                             for n in lens], dtype=object))
  for members, names, stack in groups:
    limit = 8 * int(rng.integers(4, 40))
    table_stacking.stack_tables(
        [feats[f] for f in members], names, global_device_count=local,
        num_sc_per_device=num_sc, stack_name=stack,
        stack_to_max_ids_per_partition=lambda n, b, lim=limit: lim,
        stack_to_max_unique_ids_per_partition=lambda n, b, lim=limit: lim)
  return feats, data, (weights if kind == "c3" else None)


@pytest.mark.parametrize("kind", ["c5", "c3"])
@pytest.mark.parametrize("num_sc,local", [(1, 1), (2, 1), (4, 1), (1, 2)])
@pytest.mark.parametrize("minibatching", [False, True])
def test_shapes_equal_the_oracle_buffers(kind, num_sc, local, minibatching):
  feats, data, weights = _specs(kind, 64, num_sc, local)
  got = embedding.eval_preprocess_sparse_dense_matmul_input_shape(
      feats, local, local, num_sc_per_device=num_sc,
      enable_minibatching=minibatching)
  ref = refcpu.preprocess(data, weights, feats, local, local,
                          num_sc_per_device=num_sc, allow_id_dropping=True,
                          enable_minibatching=minibatching)
  csr = got.sparse_dense_matmul_input
  assert set(csr.lhs_row_pointers) == set(ref.row_pointers)
  for field, arrays, dtype in (
      (csr.lhs_row_pointers, ref.row_pointers, np.int32),
      (csr.lhs_embedding_ids, ref.embedding_ids, np.int32),
      (csr.lhs_sample_ids, ref.sample_ids, np.int32),
      (csr.lhs_gains, ref.gains, np.float32)):
    for name, arr in arrays.items():
      assert field[name].shape == arr.shape, (name, field[name], arr.shape)
      assert field[name].dtype == dtype == arr.dtype
  assert got.num_minibatches.shape == (local,)
  assert got.num_minibatches.dtype == np.int32


def test_leading_dimension_shapes_only_the_minibatch_counts():
  """As in the reference, has_leading_dimension shapes the minibatch counts
  as (L, 1) and leaves the CSR buffers flat."""
  feats, _, _ = _specs("c3", 64, 1, 2)
  flat = embedding.eval_preprocess_sparse_dense_matmul_input_shape(
      feats, 2, 2, num_sc_per_device=1)
  lead = embedding.eval_preprocess_sparse_dense_matmul_input_shape(
      feats, 2, 2, num_sc_per_device=1, has_leading_dimension=True)
  assert lead.num_minibatches.shape == (2, 1)
  assert (lead.sparse_dense_matmul_input ==
          flat.sparse_dense_matmul_input)
  rp = flat.sparse_dense_matmul_input.lhs_row_pointers
  assert all(v.shape == (2 * 8,) for v in rp.values())
