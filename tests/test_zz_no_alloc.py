"""The allocation-free forward (scemb_sparse_dense_matmul_no_alloc); collected
last, so that a failure here hides no other test.

Called through the C ABI (ctypes) and compared with the workspace entry
point (scemb_sparse_dense_matmul) bit for bit: both run the same kernels on
the same stream, so every sum has the same order. Two calls in a row, the
second on a smaller input, for each route the forward takes: the
preprocessing's sample view (one-hot, no grouping in the call), and the CSR
alone (multi-hot, grouped by a sort inside the call, whose buffers then
live in the library's scratch array). A lookup whose workspace would exceed
the array is refused on the host before anything is enqueued.
"""

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
  if not torch.cuda.is_available():
    pytest.skip("no GPU")
  torch.cuda.set_device(0)


from jax_tpu_embedding.sparsecore import _native  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position

SCRATCH_BYTES = 64 << 20  # SCEMB_NO_ALLOC_SCRATCH_BYTES


def _batch(rng, batch, vocab, dim, valency):
  table = embedding_spec.TableSpec(
      vocabulary_size=vocab, embedding_dim=dim, initializer=None,
      optimizer=embedding_spec.SGDOptimizerSpec(0.1), combiner="sum",
      name="t", max_ids_per_partition=batch * valency,
      max_unique_ids_per_partition=batch * valency)
  feature = embedding_spec.FeatureSpec(
      table_spec=table, input_shape=[batch, valency],
      output_shape=[batch, dim], name="f")
  embedding.prepare_feature_specs_for_training([feature], 1, 1)
  ids = rng.zipf(1.2, size=(batch, valency)).astype(np.int64) % vocab
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      [ids.astype(np.int32)], None, [feature], 1, 1, num_sc_per_device=1)
  name = "t"
  keep, csr = _device.csr_operands(pre.lhs_row_pointers[name],
                                   pre.lhs_embedding_ids[name],
                                   pre.lhs_sample_ids[name],
                                   pre.lhs_gains[name], 1, 1)
  views = getattr(pre, "lookup_views", None) or {}
  table_t = torch.from_numpy(
      rng.normal(0, 1, size=(feature.table_spec.setting_in_stack
                             .padded_vocab_size, dim)).astype(np.float32)
  ).cuda()
  return keep, csr, views.get(name), table_t


def _no_alloc(csr, view, table, batch, status):
  lib = _native.load_library()
  out = torch.full((batch, table.shape[1]), float("nan"), device="cuda")
  vs = view.as_struct() if view is not None else None
  rc = lib.scemb_sparse_dense_matmul_no_alloc(
      ctypes.byref(csr), ctypes.byref(vs) if vs is not None else None,
      _native.ptr(table), int(table.shape[0]), int(table.shape[1]),
      _native.ptr(out), batch, _native.ptr(status), _native.stream_handle())
  _native.check(rc)
  return out


def _with_workspace(csr, view, table, batch, status):
  out = torch.full((batch, table.shape[1]), float("nan"), device="cuda")
  _native.sparse_dense_matmul(csr, table, out, batch, view=view,
                              device_status=status)
  return out


@pytest.mark.parametrize("use_view,valency", [(True, 1), (False, 8)])
def test_no_alloc_equals_workspace_entry(use_view, valency):
  rng = np.random.default_rng(7 + valency)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  # Two calls in a row, the second smaller: the scratch array keeps the
  # first call's contents, which the second must not depend on.
  for batch, vocab, dim in ((16384, 50000, 128), (1000, 3000, 32)):
    keep, csr, view, table = _batch(rng, batch, vocab, dim, valency)
    if use_view:
      assert view is not None
    else:
      view = None
    lib = _native.load_library()
    need = lib.scemb_sparse_dense_matmul_workspace_size(
        ctypes.byref(csr),
        ctypes.byref(view.as_struct()) if view is not None else None,
        batch, int(table.shape[0]), dim)
    assert 0 < need <= SCRATCH_BYTES
    got = _no_alloc(csr, view, table, batch, status)
    exp = _with_workspace(csr, view, table, batch, status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    np.testing.assert_array_equal(got.cpu().numpy(), exp.cpu().numpy())
    assert not np.isnan(got.cpu().numpy()).any()
    del keep


def test_no_alloc_refuses_a_lookup_beyond_its_scratch():
  """A CSR-only lookup over 4M positions needs about 100 MB of sort and
  reduction buffers: refused on the host, the output left untouched."""
  n = 1 << 22
  rp = torch.full((8,), n, dtype=torch.int32, device="cuda")
  eid = torch.zeros(n, dtype=torch.int32, device="cuda")
  sid = torch.zeros(n, dtype=torch.int32, device="cuda")
  gains = torch.ones(n, dtype=torch.float32, device="cuda")
  csr = _native.make_csr(rp, eid, sid, gains, 1, 1)
  table = torch.ones(64, 32, device="cuda")
  lib = _native.load_library()
  need = lib.scemb_sparse_dense_matmul_workspace_size(
      ctypes.byref(csr), None, 1024, 64, 32)
  assert need > SCRATCH_BYTES
  out = torch.full((1024, 32), 5.0, device="cuda")
  rc = lib.scemb_sparse_dense_matmul_no_alloc(
      ctypes.byref(csr), None, _native.ptr(table), 64, 32, _native.ptr(out),
      1024, None, _native.stream_handle())
  assert rc == _native.SCEMB_ERR_INVALID_ARGUMENT
  assert "bytes of scratch" in lib.scemb_last_error().decode()
  torch.cuda.synchronize()
  assert bool((out == 5.0).all())
