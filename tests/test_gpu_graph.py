"""The training step captured in a HIP graph (torch.cuda.CUDAGraph).

The lookup and the fused backward only launch kernels on the current stream
(no allocation, memset, copy or host wait; the workspace is the caller's), so
a whole step can be captured once and replayed. Each replay must equal the
eager step bit for bit: the test replays four times, with eager work and
synchronisations between the replays, and compares every replay's
activations, table and accumulator with an eager twin advanced step by step.
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


from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top,wrong-import-position
from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top,wrong-import-position


def _workload(one_hot, seed=0, dims=(32, 32, 32), optimizer=None,
              vocabs=(100, 5000, 70000)):
  rng = np.random.default_rng(seed)
  batch = 2048
  if optimizer is None:
    optimizer = embedding_spec.AdagradOptimizerSpec(0.05)
  tables = [embedding_spec.TableSpec(
      name=f"t{i}", vocabulary_size=int(v), embedding_dim=dims[i],
      initializer=embedding_spec.zeros,
      optimizer=optimizer, combiner="sum",
      max_ids_per_partition=1 << 16, max_unique_ids_per_partition=1 << 16)
            for i, v in enumerate(vocabs)]
  feats = [embedding_spec.FeatureSpec(
      name=f"f{i}", table_spec=t, input_shape=[batch, 1],
      output_shape=[batch, t.embedding_dim]) for i, t in enumerate(tables)]
  embedding.prepare_feature_specs_for_training(feats, 1, 1)
  ids = []
  for t in tables:
    if one_hot:
      ids.append(rng.integers(0, t.vocabulary_size, size=(batch, 1),
                              dtype=np.int32))
    else:
      rows = np.empty(batch, dtype=object)
      for i in range(batch):
        rows[i] = rng.integers(0, t.vocabulary_size,
                               size=int(rng.integers(0, 7))).astype(np.int32)
      ids.append(rows)
  pre, _ = embedding.preprocess_sparse_dense_matmul_input(
      ids, None, feats, 1, 1, num_sc_per_device=1)
  init = {}
  for name, spec in embedding.get_stacked_table_specs(feats).items():
    table = torch.tensor(rng.normal(0, 0.01, size=(
        spec.stack_vocab_size, spec.stack_embedding_dim)).astype(np.float32))
    init[name] = (table.cuda(), torch.full_like(table, 0.1).cuda())
  grads = [torch.tensor(rng.normal(size=(batch, fs.table_spec.embedding_dim)
                                   ).astype(np.float32)).cuda()
           for fs in feats]
  return feats, pre, init, grads


@pytest.mark.parametrize("dims", [(32, 32, 32), (8, 16, 32)])
@pytest.mark.parametrize("one_hot", [True, False])
def test_graph_replays_equal_eager_steps(one_hot, dims):
  """With stacks of three widths the lookups and updates run on forked side
  streams (run_per_stack), so the graph also holds their fork and join."""
  _check_graph_replays(*_workload(one_hot, dims=dims))


def test_graph_replays_with_hot_runs(monkeypatch):
  """The backward's hot-run reduction forced on (a table of 8 ids holds runs
  of hundreds of entries): its side stream's fork and join are captured
  too, and every replay equals the eager step."""
  monkeypatch.setenv("SCEMB_HOT_RUNS", "1")
  from jax_tpu_embedding.sparsecore import _native  # pylint: disable=g-import-not-at-top
  feats, pre, init, grads = _workload(False, seed=3, vocabs=(8, 5000, 70000))
  _check_graph_replays(feats, pre, init, grads)
  # The reduction ran: one eager backward with the launch spans on (not
  # during capture, which would record the spans' events into the graph).
  variables = {n: embedding.EmbeddingVariables(table=t.clone(),
                                               slot=(a.clone(),))
               for n, (t, a) in init.items()}
  _native.profile_enable(True)
  _native.profile_collect(None)
  try:
    embedding.tpu_sparse_dense_matmul_grad(
        grads, pre, variables, feats, global_device_count=1,
        num_sc_per_device=1)
    torch.cuda.synchronize()
    assert _native.profile_collect("bwd_hot_reduce")[1] > 0
  finally:
    _native.profile_collect(None)
    _native.profile_enable(False)


def _custom_adagrad(grad, table, accum, lr):
  new_accum = accum + grad * grad
  return table - lr * grad / np.sqrt(new_accum), new_accum


@pytest.mark.parametrize("mode", ["compile", "interpret"])
def test_custom_update_graph_replays_equal_eager_steps(mode, monkeypatch):
  """A custom optimizer's update captured in the graph: compiled for its
  program (the warm-up step compiles it; the capture records launches of
  the loaded code object) and interpreted."""
  monkeypatch.setenv("SCEMB_CUSTOM_UPDATE", mode)
  spec = embedding_spec.CustomOptimizerSpec(
      learning_rate=0.05, custom_computation_fn=_custom_adagrad,
      slot_variable_initializers_tuple=(lambda *_: 0.1,),
      short_name_str="custom_adagrad")
  _check_graph_replays(*_workload(False, dims=(8, 16, 32), optimizer=spec))


def _check_graph_replays(feats, pre, init, grads):

  def make_state():
    return {n: embedding.EmbeddingVariables(table=t.clone(), slot=(a.clone(),))
            for n, (t, a) in init.items()}

  def same(x, y, msg):
    for n in init:
      np.testing.assert_array_equal(x[n].table.cpu().numpy(),
                                    y[n].table.cpu().numpy(), err_msg=msg)
      np.testing.assert_array_equal(x[n].slot[0].cpu().numpy(),
                                    y[n].slot[0].cpu().numpy(), err_msg=msg)

  def step(variables):
    acts = embedding.tpu_sparse_dense_matmul(
        pre, variables, feats, global_device_count=1, num_sc_per_device=1)
    embedding.tpu_sparse_dense_matmul_grad(
        grads, pre, variables, feats, global_device_count=1,
        num_sc_per_device=1)
    return acts

  eager, graphed = make_state(), make_state()
  # Warm up on a side stream (sizes the workspace), then restore the state.
  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    step(graphed)
  torch.cuda.current_stream().wait_stream(side)
  torch.cuda.synchronize()
  for n, (t, a) in init.items():
    graphed[n].table.copy_(t)
    graphed[n].slot[0].copy_(a)
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    graph_acts = step(graphed)
  torch.cuda.synchronize()
  # Capture records without running: the state is still the initial one.
  same(graphed, make_state(), "after capture")
  for i in range(4):
    acts = step(eager)
    noise = torch.randn(1000, device="cuda").sum()  # eager work in between
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    del noise
    for a, b in zip(acts, graph_acts):
      np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy(),
                                    err_msg=f"replay {i}")
    same(eager, graphed, f"replay {i}")
