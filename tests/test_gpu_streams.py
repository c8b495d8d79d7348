"""Scratch memory across streams and graphs.

The library's workspace is one buffer per (device, stream): preprocessing
on a side stream may overlap a training step on another stream, and a
buffer a captured graph uses outlives any later growth on its stream.
Results must be bit-identical to the same work run serially.
"""

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
from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position


def _specs(batch, dim=32):
  tables = [embedding_spec.TableSpec(
      name=f"t{i}", vocabulary_size=int(v), embedding_dim=dim,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.AdagradOptimizerSpec(0.05), combiner="sum",
      max_ids_per_partition=1 << 20, max_unique_ids_per_partition=1 << 20)
            for i, v in enumerate((300, 9000, 120000))]
  feats = [embedding_spec.FeatureSpec(
      name=f"f{i}", table_spec=t, input_shape=[batch, 1],
      output_shape=[batch, dim]) for i, t in enumerate(tables)]
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  return feats


def _ids(rng, feats, multi_hot):
  out = []
  for fs in feats:
    v, b = fs.table_spec.vocabulary_size, fs.input_shape[0]
    if not multi_hot:
      out.append(rng.integers(0, v, size=(b, 1), dtype=np.int32))
      continue
    rows = np.empty(b, dtype=object)
    for i in range(b):
      rows[i] = rng.integers(0, v, size=int(rng.integers(0, 9))).astype(
          np.int32)
    out.append(rows)
  return out


def _state(feats, seed):
  rng = np.random.default_rng(seed)
  out = {}
  for name, spec in embedding.get_stacked_table_specs(feats).items():
    table = rng.normal(0, 0.01, size=(spec.stack_vocab_size,
                                      spec.stack_embedding_dim))
    out[name] = embedding.EmbeddingVariables(
        table=torch.tensor(table.astype(np.float32)).cuda(),
        slot=(torch.full((spec.stack_vocab_size, spec.stack_embedding_dim),
                         0.1, device="cuda"),))
  return out


def _clone(state):
  return {n: embedding.EmbeddingVariables(v.table.clone(),
                                          (v.slot[0].clone(),))
          for n, v in state.items()}


def _grads(feats, seed):
  rng = np.random.default_rng(seed)
  return [torch.tensor(rng.normal(size=fs.output_shape).astype(np.float32)
                       ).cuda() for fs in feats]


def _step(pre, variables, feats, grads):
  acts = embedding.tpu_sparse_dense_matmul(
      pre, variables, feats, global_device_count=1, num_sc_per_device=1)
  embedding.tpu_sparse_dense_matmul_grad(
      grads, pre, variables, feats, global_device_count=1,
      num_sc_per_device=1)
  return acts


def _csr(pre):
  return [{k: v.cpu().numpy() for k, v in d.items()}
          for d in pre.sparse_dense_matmul_input]


def _assert_same(a, b, msg):
  for n in a:
    np.testing.assert_array_equal(a[n].table.cpu().numpy(),
                                  b[n].table.cpu().numpy(), err_msg=msg)
    np.testing.assert_array_equal(a[n].slot[0].cpu().numpy(),
                                  b[n].slot[0].cpu().numpy(), err_msg=msg)


def test_each_stream_has_its_own_workspace():
  ws = _native.WORKSPACE
  a = ws.get(1 << 16)
  assert ws.get(1 << 16).data_ptr() == a.data_ptr()
  side = torch.cuda.Stream()
  with torch.cuda.stream(side):
    b = ws.get(1 << 16)
    assert ws.get(1 << 16).data_ptr() == b.data_ptr()
  assert a.data_ptr() != b.data_ptr()


@pytest.mark.parametrize("multi_hot", [False, True])
def test_preprocessing_on_a_side_stream_overlaps_steps(multi_hot):
  """Batch B is preprocessed on a side stream while steps on batch A run on
  the main stream; both equal the serial run bit for bit."""
  feats = _specs(4096)
  rng = np.random.default_rng(11)
  ids_a, ids_b = _ids(rng, feats, multi_hot), _ids(rng, feats, multi_hot)
  grads = _grads(feats, 5)
  init = _state(feats, 3)
  pre_a, _ = embedding.preprocess_sparse_dense_matmul_input(
      ids_a, None, feats, 1, 1, num_sc_per_device=1)
  # Serial reference: three steps on A, then B's preprocessing.
  serial = _clone(init)
  for _ in range(3):
    _step(pre_a, serial, feats, grads)
  pre_b_serial, _ = embedding.preprocess_sparse_dense_matmul_input(
      ids_b, None, feats, 1, 1, num_sc_per_device=1)
  torch.cuda.synchronize()
  # Overlapped: the steps are enqueued first, the side stream does not wait.
  overlapped = _clone(init)
  torch.cuda.synchronize()
  main = torch.cuda.current_stream()
  side = torch.cuda.Stream()
  for _ in range(3):
    _step(pre_a, overlapped, feats, grads)
  with torch.cuda.stream(side):
    pre_b, _ = embedding.preprocess_sparse_dense_matmul_input(
        ids_b, None, feats, 1, 1, num_sc_per_device=1)
  main.wait_stream(side)
  torch.cuda.synchronize()
  _assert_same(serial, overlapped, "steps overlapped by preprocessing")
  # Row pointers in full; the entry buffers up to the last row pointer (the
  # tail past it is left unwritten, lib/core/tests/test_utils.py:39-43).
  got, exp = _csr(pre_b), _csr(pre_b_serial)
  for name in exp[0]:
    np.testing.assert_array_equal(got[0][name], exp[0][name], err_msg=name)
    end = int(exp[0][name].max())
    for g, e in zip(got[1:], exp[1:]):
      np.testing.assert_array_equal(g[name][:end], e[name][:end],
                                    err_msg=name)


def test_graph_replays_after_its_workspace_is_outgrown():
  """A step captured on stream cs, then a larger step run eagerly on cs
  (the workspaces its calls use grow); the replays still equal an eager
  twin. The workspaces checked are those of cs and of its side streams
  (stacks of different widths would run there)."""
  small, large = _specs(512), _specs(32768, dim=128)
  rng = np.random.default_rng(21)
  pre_s, _ = embedding.preprocess_sparse_dense_matmul_input(
      _ids(rng, small, True), None, small, 1, 1, num_sc_per_device=1)
  pre_l, _ = embedding.preprocess_sparse_dense_matmul_input(
      _ids(rng, large, True), None, large, 1, 1, num_sc_per_device=1)
  g_s, g_l = _grads(small, 1), _grads(large, 2)
  init = _state(small, 4)
  eager, graphed = _clone(init), _clone(init)
  big = _state(large, 6)
  cs = torch.cuda.Stream()
  cs.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(cs):
    _step(pre_s, _clone(init), small, g_s)  # sizes cs's workspace
  torch.cuda.synchronize()
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g, stream=cs):
    graph_acts = _step(pre_s, graphed, small, g_s)
  torch.cuda.synchronize()
  dev = torch.cuda.current_device()
  sides = _native._side_streams.get((dev, cs.cuda_stream), [])  # pylint: disable=protected-access
  keys = [(dev, s.cuda_stream) for s in [cs] + list(sides)]
  bufs = _native.WORKSPACE._buf  # pylint: disable=protected-access
  captured = {k: bufs[k] for k in keys if k in bufs}
  assert captured
  with torch.cuda.stream(cs):
    _step(pre_l, big, large, g_l)  # needs larger workspaces
  torch.cuda.synchronize()
  grown = {k: bufs[k] for k in captured}
  assert any(grown[k].data_ptr() != captured[k].data_ptr() and
             grown[k].numel() > captured[k].numel() for k in captured)
  del captured, grown
  for i in range(3):
    acts = _step(pre_s, eager, small, g_s)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    for a, b in zip(acts, graph_acts):
      np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy(),
                                    err_msg=f"replay {i}")
    _assert_same(eager, graphed, f"replay {i}")


def _specs_three_stacks(batch):
  """Three tables of different dims: three stacks in one call."""
  tables = [embedding_spec.TableSpec(
      name=f"d{dim}", vocabulary_size=v, embedding_dim=dim,
      initializer=embedding_spec.zeros,
      optimizer=embedding_spec.AdagradOptimizerSpec(0.05), combiner="sum",
      max_ids_per_partition=1 << 20, max_unique_ids_per_partition=1 << 20)
            for dim, v in ((8, 700), (16, 9000), (32, 120000))]
  feats = [embedding_spec.FeatureSpec(
      name=f"f{i}", table_spec=t, input_shape=[batch, 1],
      output_shape=[batch, t.embedding_dim]) for i, t in enumerate(tables)]
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  return feats


@pytest.mark.parametrize("multi_hot", [False, True])
def test_stacks_on_side_streams_equal_one_stream(multi_hot, monkeypatch):
  """The stacks of one call are enqueued on forked side streams (the
  preprocessing, the lookups and the updates); the CSR (compared region),
  the stats and a training step equal those of the same calls with every
  stack on the calling stream."""
  feats = _specs_three_stacks(4096)
  assert len(embedding.get_stacked_table_specs(feats)) == 3
  ids = _ids(np.random.default_rng(21), feats, multi_hot)
  grads = _grads(feats, 6)
  init = _state(feats, 4)
  runs = []
  for sides in (_native.NUM_SIDE_STREAMS, 0):
    monkeypatch.setattr(_native, "NUM_SIDE_STREAMS", sides)
    pre, stats = embedding.preprocess_sparse_dense_matmul_input(
        ids, None, feats, 1, 1, num_sc_per_device=1)
    state = _clone(init)
    acts = _step(pre, state, feats, grads)
    torch.cuda.synchronize()
    runs.append((_csr(pre), stats, state,
                 [a.cpu().numpy() for a in acts]))
  (csr_a, stats_a, state_a, acts_a), (csr_b, stats_b, state_b, acts_b) = runs
  rp_a, eid_a, sid_a, gains_a = csr_a
  rp_b, eid_b, sid_b, gains_b = csr_b
  for name in rp_a:
    np.testing.assert_array_equal(rp_a[name], rp_b[name])
    end = int(rp_a[name][-1])
    for x, y in ((eid_a, eid_b), (sid_a, sid_b), (gains_a, gains_b)):
      np.testing.assert_array_equal(x[name][:end], y[name][:end],
                                    err_msg=name)
    np.testing.assert_array_equal(stats_a.max_ids_per_partition[name],
                                  stats_b.max_ids_per_partition[name])
    np.testing.assert_array_equal(stats_a.required_buffer_size_per_sc[name],
                                  stats_b.required_buffer_size_per_sc[name])
    assert stats_a.id_drop_counters[name] == stats_b.id_drop_counters[name]
  for a, b in zip(acts_a, acts_b):
    np.testing.assert_array_equal(a, b)
  _assert_same(state_a, state_b, "side streams vs one stream")


@pytest.mark.parametrize("multi_hot", [False, True])
def test_two_user_streams_preprocess_multi_stack_batches(multi_hot):
  """Two user streams each enqueue a multi-stack preprocessing (forking to
  side streams of their own) before either is waited for; each CSR and its
  stats equal the same call made alone on the default stream."""
  from jax_tpu_embedding.sparsecore.lib.core import pybind_input_preprocessing as pip  # pylint: disable=g-import-not-at-top

  feats = _specs_three_stacks(4096)
  rng = np.random.default_rng(31)
  ids = [_ids(rng, feats, multi_hot), _ids(rng, feats, multi_hot)]
  serial = []
  for batch in ids:
    *csr, pending = pip.enqueue_preprocessing(batch, None, feats, 1, 1,
                                              num_sc_per_device=1)
    serial.append((csr, pip.collect_stats(pending)))
  torch.cuda.synchronize()
  streams = [torch.cuda.Stream(), torch.cuda.Stream()]
  for s in streams:
    s.wait_stream(torch.cuda.current_stream())
  enqueued = []
  for s, batch in zip(streams, ids):
    with torch.cuda.stream(s):
      enqueued.append(pip.enqueue_preprocessing(batch, None, feats, 1, 1,
                                                num_sc_per_device=1))
  sides = [_native.side_streams(_native.NUM_SIDE_STREAMS)]
  with torch.cuda.stream(streams[0]):
    sides.append(_native.side_streams(_native.NUM_SIDE_STREAMS))
  with torch.cuda.stream(streams[1]):
    sides.append(_native.side_streams(_native.NUM_SIDE_STREAMS))
  handles = [{x.cuda_stream for x in p} for p in sides]
  assert not handles[1] & handles[2] and not handles[0] & handles[1]
  got = []
  for s, (*csr, pending) in zip(streams, enqueued):
    with torch.cuda.stream(s):
      got.append((csr, pip.collect_stats(pending)))
  torch.cuda.synchronize()
  for (csr_g, st_g), (csr_e, st_e) in zip(got, serial):
    rp_g, rp_e = csr_g[0], csr_e[0]
    for name in rp_e:
      a, b = rp_g[name].cpu().numpy(), rp_e[name].cpu().numpy()
      np.testing.assert_array_equal(a, b, err_msg=name)
      end = int(b.max())
      for x, y in zip(csr_g[1:], csr_e[1:]):
        np.testing.assert_array_equal(x[name].cpu().numpy()[:end],
                                      y[name].cpu().numpy()[:end],
                                      err_msg=name)
      np.testing.assert_array_equal(st_g.max_ids_per_partition[name],
                                    st_e.max_ids_per_partition[name])
      np.testing.assert_array_equal(st_g.required_buffer_sizes[name],
                                    st_e.required_buffer_sizes[name])
