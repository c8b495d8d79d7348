#!/usr/bin/env python3
"""Benchmark of the MI355X SparseCore embedding path.

A step is one pass of the hot path over one synthetic batch that is already
resident in HBM: the forward lookup (scemb_sparse_dense_matmul) and the
backward pass fused with the Adagrad update
(scemb_sparse_dense_matmul_grad_with_adagrad) of every stacked table. The CSR
buffers come from the GPU preprocessing, which is timed separately
(`preprocess_ms`); it also emits the sample view the forward pass consumes
and marks the CSR as sorted by row, so the step itself runs no sort. The
workload draws NUM_BATCHES seeded batches (ids, and upstream gradients
drawn on the GPU) and consecutive steps take them in turn. The
same step fed only the four reference CSR arrays (each call then sorts a
copy of the entries) is timed too (`csr_only_ms_per_step`). Default workload: the 26-table DLRM shape (one stack, dim
128, batch 65,536, one Zipf(1.1) id per feature and sample, sum combiner,
Adagrad lr 0.01 / accumulator 0.1).

Prints one JSON line (see the field comments in `main`).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "jax-tpu-embedding_amd")):
  if _p not in sys.path:
    sys.path.insert(0, _p)

METRIC = ("embedding lookups/sec + achieved HBM GB/s (fwd+bwd+Adagrad), "
          "26-table DLRM shape")
PEAK_HBM_GBS = 8000.0


def log(msg):
  print(msg, file=sys.stderr, flush=True)


def zipf_ids(rng, a, vocab, size):
  """Truncated Zipf: k ~ zipf(a), rejected when k > vocab, id = k - 1."""
  out = np.empty(size, np.int64)
  filled = 0
  while filled < size:
    k = rng.zipf(a, size=max(1024, 2 * (size - filled)))
    k = k[k <= vocab]
    take = min(size - filled, len(k))
    out[filled:filled + take] = k[:take] - 1
    filled += take
  return out.astype(np.int32)


# Distinct seeded batches a workload draws: the timed steps rotate through
# them, so no step finds the previous step's rows in the caches.
NUM_BATCHES = 4


class Workload:
  """Specs, host inputs and metadata of one benchmark configuration.
  `batches` lists (features, weights) of every drawn batch; `features` and
  `weights` are the first."""

  def __init__(self, name, feature_specs, batches, description):
    self.name = name
    self.feature_specs = feature_specs
    self.batches = batches
    self.features, self.weights = batches[0]
    self.description = description


def _batch_rngs(seed, num_batches):
  """The generator of each batch: the workload's own stream for the first
  (its specs and ids as drawn before there were several batches), seeded
  streams (seed, k) for the others."""
  return [None] + [np.random.default_rng([seed, k])
                   for k in range(1, num_batches)]


class Ragged:
  """Ragged feature: flat values plus row splits (the RaggedTensor layout
  the preprocessing accepts)."""

  def __init__(self, values, row_splits):
    self.values = values
    self.row_splits = row_splits

  def head(self, rows):
    end = int(self.row_splits[rows])
    return Ragged(self.values[:end], self.row_splits[:rows + 1])

  @property
  def size(self):
    return int(self.values.size)


def _ragged(rng, lengths, draw):
  splits = np.zeros(len(lengths) + 1, np.int64)
  np.cumsum(lengths, out=splits[1:])
  return Ragged(draw(int(splits[-1])), splits)


def _stack_all(feats, names, stack_name, limit, num_sc=1):
  from jax_tpu_embedding.sparsecore.lib.nn import table_stacking  # pylint: disable=g-import-not-at-top

  table_stacking.stack_tables(
      feats, names, global_device_count=1, num_sc_per_device=num_sc,
      stack_name=stack_name,
      stack_to_max_ids_per_partition=lambda n, b: limit,
      stack_to_max_unique_ids_per_partition=lambda n, b: limit)


def _round8(n):
  return (int(n) + 7) // 8 * 8


def c1(seed=1, num_batches=NUM_BATCHES):
  """Config 1: one table 100,000 x 16, batch 1,024, 1-16 Zipf(1.05) ids per
  sample, sum, SGD lr 0.01."""
  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top

  batch, vocab, dim = 1024, 100_000, 16
  batches = []
  for rng in _batch_rngs(seed, num_batches):
    rng = rng or np.random.default_rng(seed)
    lens = rng.integers(1, 17, size=batch)
    batches.append(([_ragged(rng, lens,
                             lambda n, r=rng: zipf_ids(r, 1.05, vocab, n))],
                    None))
  limit = _round8(max(b[0][0].size for b in batches))
  table = embedding_spec.TableSpec(
      name="t0", vocabulary_size=vocab, embedding_dim=dim,
      initializer=embedding_spec.normal(0.01),
      optimizer=embedding_spec.SGDOptimizerSpec(learning_rate=0.01),
      combiner="sum", max_ids_per_partition=limit,
      max_unique_ids_per_partition=limit)
  fs = embedding_spec.FeatureSpec(name="f0", table_spec=table,
                                  input_shape=[batch, 1],
                                  output_shape=[batch, dim])
  embedding.prepare_feature_specs_for_training([fs], 1, 1)
  return Workload("c1", [fs], batches, {
      "workload": "c1: one table 100,000 x 16, batch 1,024, 1-16 Zipf(1.05) "
                  "ids per sample, sum, SGD lr 0.01", "batch": batch})


def dlrm26(seed=0, batch=65536, num_tables=26, dim=128,
           num_batches=NUM_BATCHES):
  """Config 2 (the headline): 26 tables of dim 128, vocab log-uniform in
  [10, 4e7], batch 65,536, one Zipf(1.1) id per feature, sum, Adagrad."""
  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top

  rng = np.random.default_rng(seed)
  vocabs = np.floor(np.exp(rng.uniform(np.log(10), np.log(4e7),
                                       size=num_tables))).astype(np.int64)
  opt = embedding_spec.AdagradOptimizerSpec(learning_rate=0.01,
                                            initial_accumulator_value=0.1)
  limit = _round8(num_tables * batch)
  tables = [
      embedding_spec.TableSpec(
          name=f"t{t:02d}", vocabulary_size=int(vocabs[t]), embedding_dim=dim,
          initializer=embedding_spec.normal(0.01), optimizer=opt,
          combiner="sum", max_ids_per_partition=limit,
          max_unique_ids_per_partition=limit) for t in range(num_tables)
  ]
  feats = [
      embedding_spec.FeatureSpec(name=f"f{t:02d}", table_spec=tables[t],
                                 input_shape=[batch, 1],
                                 output_shape=[batch, dim])
      for t in range(num_tables)
  ]
  _stack_all(feats, [t.name for t in tables], "dlrm26", limit)
  batches = [([zipf_ids(r or rng, 1.1, int(vocabs[t]), batch).reshape(
      batch, 1) for t in range(num_tables)], None)
             for r in _batch_rngs(seed, num_batches)]
  return Workload(
      "dlrm26", feats, batches,
      {"workload": "dlrm26: 26 tables dim 128 stacked into one HBM buffer, "
                   "vocab log-uniform [10, 4e7] (seed 0), batch 65536, "
                   "1 Zipf(1.1) id per feature, sum, Adagrad lr 0.01",
       "tables": num_tables, "dim": dim, "batch": batch,
       "stack_rows": int(sum((v + 7) // 8 * 8 for v in vocabs))})


def c3(seed=3, num_batches=NUM_BATCHES):
  """Config 3: 8 tables 10M x 64, batch 32,768, 20-80 Zipf(1.2) ids per
  sample with U(0,1) weights; tables 0-3 sqrtn, 4-7 mean (two stacks of 40M
  rows); SGD lr 0.05."""
  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top

  batch, vocab, dim = 32768, 10_000_000, 64
  opt = embedding_spec.SGDOptimizerSpec(learning_rate=0.05)
  batches = []
  for rng in _batch_rngs(seed, num_batches):
    rng = rng or np.random.default_rng(seed)
    features, weights = [], []
    for t in range(8):
      lens = rng.integers(20, 81, size=batch)
      f = _ragged(rng, lens, lambda n, r=rng: zipf_ids(r, 1.2, vocab, n))
      features.append(f)
      weights.append(Ragged(
          rng.uniform(0, 1, size=f.size).astype(np.float32), f.row_splits))
    batches.append((features, weights))
  feats, tables = [], []
  for t in range(8):
    tables.append(embedding_spec.TableSpec(
        name=f"t{t}", vocabulary_size=vocab, embedding_dim=dim,
        initializer=embedding_spec.normal(0.01), optimizer=opt,
        combiner="sqrtn" if t < 4 else "mean", max_ids_per_partition=1,
        max_unique_ids_per_partition=1))
    feats.append(embedding_spec.FeatureSpec(
        name=f"f{t}", table_spec=tables[-1], input_shape=[batch, 1],
        output_shape=[batch, dim]))
  for k, group in enumerate((range(0, 4), range(4, 8))):
    limit = _round8(max(sum(b[0][t].size for t in group) for b in batches))
    _stack_all([feats[t] for t in group], [f"t{t}" for t in group],
               f"c3_{'sqrtn' if k == 0 else 'mean'}", limit)
  return Workload("c3", feats, batches, {
      "workload": "c3: 8 tables 10M x 64 in two stacks (sqrtn, mean), batch "
                  "32,768, 20-80 Zipf(1.2) ids per sample, U(0,1) weights, "
                  "SGD lr 0.05", "batch": batch})


def c4(seed=4, num_batches=NUM_BATCHES):
  """Config 4: one table 200M x 128 (102 GB, plus a 102 GB accumulator),
  batch 131,072, 50 Zipf(1.3) ids per sample, sum, Adagrad."""
  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top

  batch, vocab, dim, k = 131072, 200_000_000, 128, 50
  batches = [([zipf_ids(r or np.random.default_rng(seed), 1.3, vocab,
                        batch * k).reshape(batch, k)], None)
             for r in _batch_rngs(seed, num_batches)]
  table = embedding_spec.TableSpec(
      name="t0", vocabulary_size=vocab, embedding_dim=dim,
      initializer=embedding_spec.normal(0.01),
      optimizer=embedding_spec.AdagradOptimizerSpec(
          learning_rate=0.01, initial_accumulator_value=0.1),
      combiner="sum", max_ids_per_partition=_round8(batch * k),
      max_unique_ids_per_partition=_round8(batch * k))
  fs = embedding_spec.FeatureSpec(name="f0", table_spec=table,
                                  input_shape=[batch, k],
                                  output_shape=[batch, dim])
  embedding.prepare_feature_specs_for_training([fs], 1, 1)
  return Workload("c4", [fs], batches, {
      "workload": "c4: one table 200M x 128 (102 GB + 102 GB accumulator), "
                  "batch 131,072, 50 Zipf(1.3) ids per sample, sum, Adagrad",
      "batch": batch})


def c5(seed=5, num_batches=NUM_BATCHES):
  """Config 5: 40 features over 12 tables (dims 8..256, vocab log-uniform
  [1e4, 5e6]), power-law lengths on [1, 500], uniform ids on tables 0-5 and
  Zipf(1.05) on 6-11, batch 16,384, mean, Adagrad; six stacks (one per
  dim) with feature stacking."""
  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top

  rng = np.random.default_rng(seed)
  batch = 16384
  dims = [8, 16, 32, 64, 128, 256]
  vocabs = np.floor(np.exp(rng.uniform(np.log(1e4), np.log(5e6),
                                       size=12))).astype(np.int64)
  opt = embedding_spec.AdagradOptimizerSpec(learning_rate=0.01,
                                            initial_accumulator_value=0.1)
  support = np.arange(1, 501)
  p = support.astype(np.float64) ** -1.5
  p /= p.sum()
  tables = [embedding_spec.TableSpec(
      name=f"t{t:02d}", vocabulary_size=int(vocabs[t]),
      embedding_dim=dims[t % 6], initializer=embedding_spec.normal(0.01),
      optimizer=opt, combiner="mean", max_ids_per_partition=1,
      max_unique_ids_per_partition=1) for t in range(12)]
  batches = []
  for r in _batch_rngs(seed, num_batches):
    r = r or rng
    features = []
    for f in range(40):
      t = f % 12
      lens = r.choice(support, size=batch, p=p)
      if t < 6:
        draw = lambda n, v=int(vocabs[t]), r=r: r.integers(
            0, v, size=n).astype(np.int32)
      else:
        draw = lambda n, v=int(vocabs[t]), r=r: zipf_ids(r, 1.05, v, n)
      features.append(_ragged(r, lens, draw))
    batches.append((features, None))
  feats = []
  for f in range(40):
    t = f % 12
    feats.append(embedding_spec.FeatureSpec(
        name=f"f{f:02d}", table_spec=tables[t], input_shape=[batch, 1],
        output_shape=[batch, dims[t % 6]]))
  for d in range(6):
    group = [f for f in range(40) if f % 12 in (d, d + 6)]
    limit = _round8(max(sum(b[0][f].size for f in group) for b in batches))
    _stack_all([feats[f] for f in group], [f"t{d:02d}", f"t{d + 6:02d}"],
               f"c5_d{dims[d]}", limit)
  return Workload("c5", feats, batches, {
      "workload": "c5: 40 features over 12 tables (dims 8-256, vocab "
                  "log-uniform [1e4, 5e6]) in six stacks, power-law lengths "
                  "[1, 500], batch 16,384, mean, Adagrad", "batch": batch})


WORKLOADS = {"c1": c1, "c2": dlrm26, "c3": c3, "c4": c4, "c5": c5}


def copy_probe(dev, gib=1):
  """A plain device copy of `gib` GiB, three times: the calibration kernel
  for the FETCH_SIZE / WRITE_SIZE counters (each launch must read and write
  exactly gib GiB)."""
  import torch  # pylint: disable=g-import-not-at-top

  n = gib * (1 << 30) // 4
  a = torch.ones(n, dtype=torch.float32, device=dev)
  b = torch.empty_like(a)
  for _ in range(3):
    b.copy_(a)
  torch.cuda.synchronize()
  log(f"copy probe: 3 x {gib} GiB device copies")
  del a, b


def copy_rate_gbs(dev, gib=1, reps=5):
  """HBM bytes per second of a plain device copy of `gib` GiB (read plus
  write), median of `reps` event-timed copies: the rate a bandwidth-bound
  kernel of this mix can reach on this box, measured in the same run."""
  import torch  # pylint: disable=g-import-not-at-top

  n = gib * (1 << 30) // 4
  a = torch.ones(n, dtype=torch.float32, device=dev)
  b = torch.empty_like(a)
  b.copy_(a)
  times = []
  for _ in range(reps):
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    b.copy_(a)
    e1.record()
    e1.synchronize()
    times.append(e0.elapsed_time(e1) / 1e3)
  del a, b
  torch.cuda.empty_cache()
  return 2 * gib * (1 << 30) / float(np.median(times)) / 1e9


def _stack_batch_ids(w: Workload, features=None):
  """Input ids (lookups) per stack of one batch (the first by default)."""
  out = {}
  for f, fs in zip(w.features if features is None else features,
                   w.feature_specs):
    name = fs.table_spec.stacked_table_spec.stack_name
    out[name] = out.get(name, 0) + int(np.asarray(f).size if not isinstance(
        f, Ragged) else f.size)
  return out


def run_gpu(w: Workload, steps: int, warmup: int, probe: bool = False,
            api: bool = True, other_optimizers: bool = True,
            minibatching: bool = True):
  import torch  # pylint: disable=g-import-not-at-top

  from jax_tpu_embedding.sparsecore import _native  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr as fwd  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as ada  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_sgd as sgd  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top

  torch.cuda.set_device(0)
  dev = torch.device("cuda", 0)
  if probe:
    copy_probe(dev)
  copy_gbs = copy_rate_gbs(dev)
  log(f"device copy: {copy_gbs:.1f} GB/s")
  stacked = embedding.get_stacked_table_specs(w.feature_specs)

  def resident(x):
    if isinstance(x, Ragged):
      return Ragged(torch.from_numpy(np.asarray(x.values)).to(dev),
                    x.row_splits)
    return torch.from_numpy(np.asarray(x)).to(dev)

  # Inputs of every batch resident in HBM before anything is timed.
  inputs_dev = []
  for feats, weights in w.batches:
    inputs_dev.append(([resident(f) for f in feats],
                       None if weights is None else
                       [resident(x) for x in weights]))
  feats_dev, weights_dev = inputs_dev[0]
  nb = len(inputs_dev)
  torch.cuda.synchronize()

  def preprocess(k, enqueue=False):
    fn = (embedding.enqueue_preprocess_sparse_dense_matmul_input if enqueue
          else embedding.preprocess_sparse_dense_matmul_input)
    return fn(*inputs_dev[k % nb], w.feature_specs, 1, 1,
              num_sc_per_device=1)

  # GPU preprocessing (reported separately): median of 5 after 2 warmups,
  # each call on the next batch.
  pre_times = []
  for i in range(7):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    preprocess(i)
    torch.cuda.synchronize()
    if i >= 2:
      pre_times.append(time.perf_counter() - t0)
  preprocess_ms = float(np.median(pre_times) * 1e3)
  log(f"preprocess: {preprocess_ms:.3f} ms (median of {len(pre_times)})")
  pres = [preprocess(k) for k in range(nb)]
  pre, stats = pres[0]
  pres = [p for p, _ in pres]
  gen = torch.Generator(device=dev)
  gen.manual_seed(1234)
  state = {}
  grads = [{} for _ in range(nb)]
  per_stack = {}
  ids = [_stack_batch_ids(w, feats) for feats, _ in w.batches]
  for name, spec in stacked.items():
    rows, dim = spec.stack_vocab_size, spec.stack_embedding_dim
    t = torch.empty((rows, dim), dtype=torch.float32, device=dev)
    t.normal_(0.0, 0.01, generator=gen)
    adagrad = isinstance(spec.optimizer, embedding_spec.AdagradOptimizerSpec)
    a = None
    if adagrad:
      a = torch.full((rows, dim), spec.optimizer.initial_accumulator_value,
                     dtype=torch.float32, device=dev)
    bs = spec.total_sample_count
    for k in range(nb):
      g = torch.empty((bs, dim), dtype=torch.float32, device=dev)
      g.normal_(0.0, 1.0, generator=gen)
      grads[k][name] = g
    lr = torch.tensor(spec.optimizer.learning_rate, dtype=torch.float32,
                      device=dev)
    state[name] = (t, a, grads[0][name], lr)
    # Entries and distinct rows of each batch; the compulsory bytes use
    # their means over the batches the steps rotate through.
    ns, us = [], []
    for p in pres:
      rp = p.lhs_row_pointers[name].cpu().numpy()
      n_valid = int(rp[0])  # one partition (S = NS = 1)
      ns.append(n_valid)
      us.append(int(torch.unique(p.lhs_embedding_ids[name][:n_valid]).numel()))
    per_stack[name] = {"N": float(np.mean(ns)), "U": float(np.mean(us)),
                       "Bs": bs, "D": dim, "rows": rows,
                       "ids": float(np.mean([x[name] for x in ids])),
                       "optimizer": "adagrad" if adagrad else "sgd",
                       "N_per_batch": ns, "U_per_batch": us}
    log(f"stack {name}: rows={rows} dim={dim} N={ns} U={us} Bs={bs}")
  lookups = float(np.mean([sum(x.values()) for x in ids]))

  def step(csr_only=False, batch=None, k=0):
    """One step on batch k (its CSR and upstream gradients); `batch`, if
    given, is a PreprocessedInput of batch k made elsewhere."""
    p = pres[k % nb] if batch is None else batch
    grad = grads[k % nb]

    def csr_of(name):
      return (p.lhs_row_pointers[name], p.lhs_embedding_ids[name],
              p.lhs_sample_ids[name], p.lhs_gains[name])

    def lookup(name):
      spec = stacked[name]
      return fwd.tpu_sparse_dense_matmul_csr_primitive.bind(
          *csr_of(name), 1, state[name][0],
          device_batch_size=spec.total_sample_count,
          max_ids_per_partition=spec.max_ids_per_partition,
          max_unique_ids_per_partition=spec.max_unique_ids_per_partition,
          num_sc_per_device=1,
          lookup_view=None if csr_only else p.lookup_views[name],
          csr_num_entries=None if csr_only else
          (p.csr_num_entries or {}).get(name))

    def update(name):
      spec = stacked[name]
      t, a, _, lr = state[name]
      g = grad[name]
      kw = dict(max_ids_per_partition=spec.max_ids_per_partition,
                max_unique_ids_per_partition=spec.max_unique_ids_per_partition,
                num_sc_per_device=1,
                csr_sorted_by_row=None if csr_only else
                p.csr_sorted_by_row,
                csr_num_entries=None if csr_only else
                (p.csr_num_entries or {}).get(name))
      if a is not None:
        return ada.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
            *csr_of(name), 1, t, a, g, lr, **kw)
      return sgd.tpu_sparse_dense_matmul_grad_with_sgd_primitive.bind(
          *csr_of(name), 1, t, g, lr, **kw)

    # The order of a training step: the lookups of every stack, then their
    # updates; stacks of different widths run concurrently on side streams,
    # as the embedding API runs them (one width runs inline).
    width = lambda n: stacked[n].stack_embedding_dim
    _native.run_per_stack(stacked.keys(), lookup, width)
    _native.run_per_stack(stacked.keys(), update, width)

  def timed(n, csr_only, rotate=True):
    """ms per step over n steps, batch i % nb at step i (batch 0 at every
    step without `rotate`)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
      step(csr_only, k=i if rotate else 0)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / n

  for i in range(warmup):
    step(True, k=i)
  csr_only_ms = timed(steps, True)
  log(f"step with the reference CSR arrays only: {csr_only_ms:.4f} ms")
  for i in range(warmup):
    step(k=i)
  ms_per_step = timed(steps, False)
  log(f"step, {nb} batches in turn: {ms_per_step:.4f} ms")
  same_batch_ms = timed(steps, False, rotate=False)
  log(f"step, one batch at every step: {same_batch_ms:.4f} ms")
  graph_ms = _graph_steps(step, steps, warmup)
  log(f"step replayed from a HIP graph: {graph_ms:.4f} ms")
  pipelined_ms = _pipelined_steps(
      step, lambda k: preprocess(k, enqueue=True), steps, warmup)
  log(f"step with the next batch preprocessed alongside: "
      f"{pipelined_ms:.4f} ms")
  # Kernel durations from HIP events on the launch stream, in a second pass
  # of the same steps (the events themselves cost a few microseconds each,
  # so the timed pass above runs without them). Stacks run one after another
  # in this pass: side by side, each event pair would also span the other
  # stacks' kernels sharing the GPU.
  sides = _native.NUM_SIDE_STREAMS
  _native.NUM_SIDE_STREAMS = 0
  _native.profile_enable(True)
  _native.profile_collect(None)
  timed(steps, False)
  _native.profile_enable(False)
  _native.NUM_SIDE_STREAMS = sides
  api_ms = api_copy_ms = None
  if api:
    api_ms, api_copy_ms = _api_steps(w, pre, state, stacked, steps, warmup,
                                     timed_fn=torch.cuda.synchronize)
    log(f"API step (per-feature tensors): fused stacking {api_ms:.4f} ms, "
        f"with stacking copies {api_copy_ms:.4f} ms")
  opt_ms = None
  if other_optimizers and len(stacked) == 1:
    opt_ms = _optimizer_steps(pre, state, stacked, steps, warmup)
    log("backward + optimizer: " + ", ".join(
        f"{k} {v:.4f} ms" for k, v in opt_ms.items()))
  mb = None
  if minibatching and len(stacked) == 1:
    mb = _minibatching_steps(w, feats_dev, weights_dev, state, stacked,
                             steps, warmup)
    log(f"minibatching ({mb['num_minibatches']} minibatches): preprocess "
        f"{mb['preprocess_ms']:.3f} ms, step {mb['ms_per_step']:.4f} ms, "
        f"dropped {mb['dropped']}")
  spans = {}
  for k in ("fwd_reduce", "fwd_finish", "bwd_reduce", "bwd_finish",
            "bwd_hot_plan", "bwd_hot_reduce", "fwd_call", "bwd_call"):
    ms, n = _native.profile_collect(k)
    # Per step, summed over the stacks (one launch per stack and step).
    spans[k] = (ms / steps if n else 0.0, n)
  log(f"step: {ms_per_step:.4f} ms; per-step spans " +
      ", ".join(f"{k} {v[0]:.4f}" for k, v in spans.items()))
  return {
      "api_ms_per_step": api_ms,
      "api_copy_ms_per_step": api_copy_ms,
      "csr_only_ms_per_step": csr_only_ms,
      "ms_per_step": ms_per_step,
      "same_batch_ms_per_step": same_batch_ms,
      "num_batches": nb,
      "graph_ms_per_step": graph_ms,
      "pipelined_ms_per_step": pipelined_ms,
      "lookups": lookups,
      "preprocess_ms": preprocess_ms,
      "spans": spans,
      "per_stack": per_stack,
      "dropped": int(sum(stats.id_drop_counters.values())),
      "optimizer_bwd_ms": opt_ms,
      "minibatching": mb,
      "copy_gbs": copy_gbs,
  }


def _device_tensors(obj, out):
  """The torch tensors reachable from a PreprocessedInput (dicts, lists,
  dataclass-like objects)."""
  import torch  # pylint: disable=g-import-not-at-top

  if isinstance(obj, torch.Tensor):
    out.append(obj)
  elif isinstance(obj, dict):
    for v in obj.values():
      _device_tensors(v, out)
  elif isinstance(obj, (list, tuple)):
    for v in obj:
      _device_tensors(v, out)
  elif hasattr(obj, "__dict__"):
    for v in vars(obj).values():
      _device_tensors(v, out)
  return out


def _pipelined_steps(step, preprocess, steps, warmup):
  """Steady state of a training loop that preprocesses batch k + 1 on a
  second stream while step k runs: each iteration enqueues step k on the
  current stream, enqueues the preprocessing of the next batch (the next of
  the synthetic inputs in HBM, `preprocess(k + 1)`) on the side stream
  (enqueue_preprocess_sparse_dense_matmul_input), then collects batch k's
  stats, whose copy finished before step k could start; the next step waits
  for the side stream. The host never waits for the step. ms per step."""
  import torch  # pylint: disable=g-import-not-at-top

  main = torch.cuda.current_stream()
  side = torch.cuda.Stream()

  def next_batch(k):
    with torch.cuda.stream(side):
      b, stats = preprocess(k)
    # The batch is consumed on the main stream: its memory must not return
    # to the side stream's pool before the main stream is done with it.
    for t in _device_tensors(b, []):
      t.record_stream(main)
    main.wait_stream(side)
    return b, stats

  k = 0
  cur, stats = next_batch(k)
  for _ in range(warmup):
    step(False, cur, k)
    nxt = next_batch(k + 1)
    stats.result()
    cur, stats = nxt
    k += 1
  torch.cuda.synchronize()
  t0 = time.perf_counter()
  for _ in range(steps):
    step(False, cur, k)
    nxt = next_batch(k + 1)
    stats.result()
    cur, stats = nxt
    k += 1
  torch.cuda.synchronize()
  stats.result()
  return (time.perf_counter() - t0) * 1e3 / steps


def _graph_steps(step, steps, warmup):
  """The same step captured once in a HIP graph (torch.cuda.CUDAGraph) and
  replayed: the kernels of a step, without the host work of each call (the
  step only launches kernels, so it captures as is). ms per replay."""
  import torch  # pylint: disable=g-import-not-at-top

  side = torch.cuda.Stream()
  side.wait_stream(torch.cuda.current_stream())
  with torch.cuda.stream(side):
    step()
  torch.cuda.current_stream().wait_stream(side)
  g = torch.cuda.CUDAGraph()
  with torch.cuda.graph(g):
    step()
  for _ in range(warmup):
    g.replay()
  torch.cuda.synchronize()
  t0 = time.perf_counter()
  for _ in range(steps):
    g.replay()
  torch.cuda.synchronize()
  ms = (time.perf_counter() - t0) * 1e3 / steps
  del g
  return ms


# Every built-in optimizer spec with two slot variables, at its defaults.
OTHER_OPTIMIZERS = ("adam", "adagrad_momentum", "ftrl", "laprop", "f2a")
# The optimizer_bwd entries with one slot variable (the others have two).
ONE_SLOT_OPTIMIZERS = ("adagrad", "custom_adagrad", "custom_adagrad_interpreted")


def _optimizer_steps(pre, state, stacked, steps, warmup):
  """Backward + Adagrad (built-in and custom) and each two-slot optimizer on
  the headline stack (the step's backward with another update): ms per call, event-free wall time over
  `steps` calls. Slots start at the spec's initial values; the table is the
  step's own (updated in place, as in training)."""
  import torch  # pylint: disable=g-import-not-at-top

  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top

  specs = {
      "adam": embedding_spec.AdamOptimizerSpec(learning_rate=0.001),
      "adagrad_momentum": embedding_spec.AdagradMomentumOptimizerSpec(
          learning_rate=0.01),
      "ftrl": embedding_spec.FTRLOptimizerSpec(learning_rate=0.01),
      "laprop": embedding_spec.LaPropOptimizerSpec(learning_rate=0.001),
      "f2a": embedding_spec.F2AOptimizerSpec(learning_rate=0.01),
  }
  (name, spec), = stacked.items()
  t, _, g, _ = state[name]
  slots = [torch.empty_like(t), torch.empty_like(t)]
  csr = (pre.lhs_row_pointers[name], pre.lhs_embedding_ids[name],
         pre.lhs_sample_ids[name], pre.lhs_gains[name])
  kw = dict(max_ids_per_partition=spec.max_ids_per_partition,
            max_unique_ids_per_partition=spec.max_unique_ids_per_partition,
            num_sc_per_device=1, csr_sorted_by_row=pre.csr_sorted_by_row,
            csr_num_entries=pre.csr_num_entries[name])
  out = {}
  # The reference test's custom Adagrad (tpu_sparse_dense_matmul_grad_test.py:
  # 1324-1486) beside the built-in Adagrad (the same bytes, one slot): its
  # update compiled for the program at run time (compiled once, in the
  # warmup), and interpreted.
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_optimizer_grad as custom  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as ada  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import custom_optimizer_lowering  # pylint: disable=g-import-not-at-top

  def adagrad_fn(grad, table, accum, lr):
    new_accum = accum + grad * grad
    return table - lr * grad / np.sqrt(new_accum), new_accum

  text = custom_optimizer_lowering.lower_to_stablehlo(
      adagrad_fn, int(t.shape[1]), 1, 1)
  lr = torch.tensor(0.01, dtype=torch.float32, device=t.device)
  acc = slots[0]
  def custom_call():
    custom.tpu_sparse_dense_matmul_optimizer_grad_primitive.bind(
        *csr, 1, g, lr, t, acc, num_hyperparameters=1, stablehlo=text, **kw)

  variants = {
      "adagrad": (None, lambda: ada.tpu_sparse_dense_matmul_grad_with_adagrad_primitive
                  .bind(*csr, 1, t, acc, g, lr, **kw)),
      "custom_adagrad": ("compile", custom_call),
      "custom_adagrad_interpreted": ("interpret", custom_call),
  }
  saved_mode = os.environ.get("SCEMB_CUSTOM_UPDATE")
  for key, (mode, call) in variants.items():
    if mode is not None:
      os.environ["SCEMB_CUSTOM_UPDATE"] = mode
    acc.fill_(0.1)
    for _ in range(warmup):
      call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
      call()
    torch.cuda.synchronize()
    out[key] = (time.perf_counter() - t0) * 1e3 / steps
  if saved_mode is None:
    os.environ.pop("SCEMB_CUSTOM_UPDATE", None)
  else:
    os.environ["SCEMB_CUSTOM_UPDATE"] = saved_mode
  for key in OTHER_OPTIMIZERS:
    opt = specs[key]
    for s, init in zip(slots, opt.slot_variables_initializers()):
      s.fill_(init.constant_value)
    hyper = [h if isinstance(h, (bool, np.bool_)) else
             torch.tensor(float(h), dtype=torch.float32, device=t.device)
             for h in opt.get_hyperparameters(0)]
    extra = ({"multiply_linear_by_learning_rate":
              opt.multiply_linear_by_learning_rate}
             if key == "ftrl" else {})
    prim = opt.get_optimizer_primitive()

    def call():
      prim.bind(*csr, 1, t, *slots, g, *hyper, **kw, **extra)  # pylint: disable=cell-var-from-loop

    for _ in range(warmup):
      call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
      call()
    torch.cuda.synchronize()
    out[key] = (time.perf_counter() - t0) * 1e3 / steps
  del slots
  torch.cuda.empty_cache()
  return out


# Stack limit for the minibatching leg: at the headline shape (1.7M entries
# in one partition) it splits the 64 buckets into several minibatches without
# dropping an id.
MINIBATCH_LIMIT = 1 << 18


def _minibatching_steps(w, feats_dev, weights_dev, state, stacked, steps,
                        warmup):
  """The headline stack with enable_minibatching and limits of
  MINIBATCH_LIMIT ids per partition: the three-pass preprocessing (median of
  5 after 2 warmups, host time including its two device waits) and the
  forward + Adagrad step over the minibatched CSR (the forward from the
  preprocessing's sample view, the backward reading the CSR in place)."""
  import torch  # pylint: disable=g-import-not-at-top

  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_csr as fwd  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.core.primitives import sparse_dense_matmul_grad_with_adagrad as ada  # pylint: disable=g-import-not-at-top
  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top

  (name, spec), = stacked.items()
  saved = [fs.table_spec.stacked_table_spec for fs in w.feature_specs]
  for fs, st in zip(w.feature_specs, saved):
    fs.table_spec.stacked_table_spec = st.replace(
        max_ids_per_partition=MINIBATCH_LIMIT,
        max_unique_ids_per_partition=MINIBATCH_LIMIT,
        suggested_coo_buffer_size_per_device=None)
  try:
    times = []
    for i in range(7):
      torch.cuda.synchronize()
      t0 = time.perf_counter()
      pre, stats = embedding.preprocess_sparse_dense_matmul_input(
          feats_dev, weights_dev, w.feature_specs, 1, 1, num_sc_per_device=1,
          enable_minibatching=True)
      torch.cuda.synchronize()
      if i >= 2:
        times.append(time.perf_counter() - t0)
  finally:
    for fs, st in zip(w.feature_specs, saved):
      fs.table_spec.stacked_table_spec = st
  nmb = int(pre.num_minibatches[0])
  t, a, g, lr = state[name]
  csr = (pre.lhs_row_pointers[name], pre.lhs_embedding_ids[name],
         pre.lhs_sample_ids[name], pre.lhs_gains[name])
  kw = dict(max_ids_per_partition=MINIBATCH_LIMIT,
            max_unique_ids_per_partition=MINIBATCH_LIMIT, num_sc_per_device=1,
            enable_minibatching=True,
            csr_num_entries=pre.csr_num_entries[name])

  def step():
    fwd.tpu_sparse_dense_matmul_csr_primitive.bind(
        *csr, nmb, t, device_batch_size=spec.total_sample_count,
        lookup_view=pre.lookup_views[name], **kw)
    ada.tpu_sparse_dense_matmul_grad_with_adagrad_primitive.bind(
        *csr, nmb, t, a, g, lr, csr_sorted_by_row=pre.csr_sorted_by_row, **kw)

  for _ in range(warmup):
    step()
  torch.cuda.synchronize()
  t0 = time.perf_counter()
  for _ in range(steps):
    step()
  torch.cuda.synchronize()
  ms = (time.perf_counter() - t0) * 1e3 / steps
  return {"num_minibatches": nmb,
          "max_ids_per_partition": MINIBATCH_LIMIT,
          "preprocess_ms": float(np.median(times) * 1e3),
          "ms_per_step": ms,
          "dropped": int(sum(stats.id_drop_counters.values()))}


def _api_steps(w, pre, state, stacked, steps, warmup, timed_fn):
  """The same step through the embedding API with per-feature activations
  and gradients (what a training loop sees): once with the stacking fused
  into the kernels (the default), once with the stacked-matrix path and the
  unstack / stack copies. Returns (fused ms, copy ms) per step."""
  import torch  # pylint: disable=g-import-not-at-top

  from jax_tpu_embedding.sparsecore.lib.nn import embedding  # pylint: disable=g-import-not-at-top

  specs = w.feature_specs
  variables = {}
  grads = []
  for name in stacked:
    t, a, _, _ = state[name]
    variables[name] = embedding.EmbeddingVariables(
        t, (a,) if a is not None else ())
  for fs in specs:
    _, _, g, _ = state[fs.table_spec.stacked_table_spec.stack_name]
    rows = fs.output_shape[0]
    off = fs.id_transformation.row_offset
    grads.append(g[off:off + rows, :fs.table_spec.embedding_dim].contiguous())

  def fused():
    embedding.tpu_sparse_dense_matmul(pre, variables, specs,
                                      global_device_count=1,
                                      num_sc_per_device=1)
    embedding.tpu_sparse_dense_matmul_grad(grads, pre, variables, specs,
                                           global_device_count=1,
                                           num_sc_per_device=1)

  def copies():
    acts = embedding.tpu_sparse_dense_matmul(
        pre, variables, specs, global_device_count=1, num_sc_per_device=1,
        perform_unstacking=False)
    outs = embedding.unstack_embedding_activations(acts, specs, 1, 1)
    for o in outs:  # a training loop consumes contiguous activations
      o.contiguous()
    sg = embedding.stack_embedding_gradients(grads, specs, 1)
    embedding.tpu_sparse_dense_matmul_grad(
        sg, pre, variables, specs, global_device_count=1,
        num_sc_per_device=1, perform_stacking=False)

  out = []
  for fn in (fused, copies):
    for _ in range(warmup):
      fn()
    timed_fn()
    t0 = time.perf_counter()
    for _ in range(steps):
      fn()
    timed_fn()
    out.append((time.perf_counter() - t0) * 1e3 / steps)
  del torch
  return tuple(out)


def algorithmic_bytes(per_stack):
  """Compulsory HBM bytes of the forward and of backward + optimizer."""
  fwd = bwd = 0
  for s in per_stack.values():
    n, u, bs, d = s["N"], s["U"], s["Bs"], s["D"]
    fwd += 12 * n + 4 * d * u + 4 * d * bs
    slot = 16 if s["optimizer"] == "adagrad" else 8
    bwd += 12 * n + 4 * d * bs + slot * d * u
  return fwd, bwd


def _head(x, rows):
  if isinstance(x, Ragged):
    return x.head(rows)
  return np.asarray(x)[:rows]


def cpu_baseline(w: Workload, sample_batch: int, seconds: float,
                 minibatching: bool = False):
  """The oracle (C++ restatement of the reference CPU path) on host cores,
  on the first `sample_batch` samples of every feature."""
  import copy  # pylint: disable=g-import-not-at-top

  from jax_tpu_embedding.sparsecore.lib.nn import embedding_spec  # pylint: disable=g-import-not-at-top
  from oracle import refcpu  # pylint: disable=g-import-not-at-top

  # A one-GPU box's CPU share is 16 cores, whatever the host has in all.
  threads = min(CPU_SHARE, _usable_cpus())
  batch = w.feature_specs[0].input_shape[0]
  sample_batch = min(sample_batch, batch)
  feats = [_head(f, sample_batch) for f in w.features]
  weights = (None if w.weights is None else
             [_head(x, sample_batch) for x in w.weights])
  # The oracle takes per-sample arrays for ragged input.
  def rows(x):
    if not isinstance(x, Ragged):
      return x
    out = np.empty(len(x.row_splits) - 1, dtype=object)
    for i in range(len(out)):
      out[i] = np.asarray(x.values[x.row_splits[i]:x.row_splits[i + 1]])
    return out
  feats = [rows(f) for f in feats]
  weights = None if weights is None else [rows(x) for x in weights]
  # Same stacking geometry with the sample's batch: each feature keeps its
  # slot in the stack, its row offset scales with the batch.
  specs = []
  for fs in w.feature_specs:
    nfs = copy.copy(fs)
    nfs.input_shape = [sample_batch] + list(fs.input_shape[1:])
    tr = fs.id_transformation
    slot = tr.row_offset // fs.input_shape[0]
    nfs._id_transformation = embedding_spec.FeatureIdTransformation(  # pylint: disable=protected-access
        row_offset=slot * sample_batch, col_offset=tr.col_offset,
        col_shift=tr.col_shift)
    specs.append(nfs)
  stacked = {}
  for fs in specs:
    st = fs.table_spec.stacked_table_spec
    stacked[st.stack_name] = st
  t0 = time.perf_counter()
  ref = refcpu.preprocess(feats, weights, specs, 1, 1, num_sc_per_device=1)
  pre_s = time.perf_counter() - t0
  mb = None
  if minibatching and len(stacked) == 1:
    # The minibatching passes on the sample, with the limit scaled to the
    # sample so that the split is alike.
    limit = max(8, MINIBATCH_LIMIT * sample_batch // batch)
    mb_specs = []
    for fs in specs:
      nfs = copy.copy(fs)
      nfs.table_spec = copy.copy(fs.table_spec)
      nfs.table_spec.stacked_table_spec = (
          fs.table_spec.stacked_table_spec.replace(
              max_ids_per_partition=limit, max_unique_ids_per_partition=limit,
              suggested_coo_buffer_size_per_device=None))
      mb_specs.append(nfs)
    t0 = time.perf_counter()
    mb_ref = refcpu.preprocess(feats, weights, mb_specs, 1, 1,
                               num_sc_per_device=1, enable_minibatching=True)
    mb = (time.perf_counter() - t0, mb_ref.num_minibatches, limit)
  total_lookups = sum(int(f.size) if not isinstance(f, np.ndarray) or
                      f.dtype != object else sum(len(r) for r in f)
                      for f in feats)
  busy = 0.0
  iters = 0
  rng = np.random.default_rng(5)
  state = {}
  for name, st in stacked.items():
    rows_, dim = st.stack_vocab_size, st.stack_embedding_dim
    # calloc'd: only the rows the sample touches are ever paged in.
    table = np.zeros((rows_, dim), np.float32)
    adagrad = isinstance(st.optimizer, embedding_spec.AdagradOptimizerSpec)
    acc = np.zeros((rows_, dim), np.float32) if adagrad else None
    n = int(ref.row_pointers[name][0])
    touched = np.unique(ref.embedding_ids[name][:n])
    table[touched] = rng.normal(0, 0.01, size=(len(touched), dim))
    if adagrad:
      acc[touched] = st.optimizer.initial_accumulator_value
    bs = sum(1 for fs in specs
             if fs.table_spec.stacked_table_spec.stack_name == name
             ) * sample_batch
    grad = rng.normal(0, 1, size=(bs, dim)).astype(np.float32)
    state[name] = (table, acc, grad, bs, st.optimizer.learning_rate)
  while busy < seconds or iters < 3:
    t0 = time.perf_counter()
    for name in stacked:
      table, acc, grad, bs, lr = state[name]
      args = (ref.row_pointers[name], ref.embedding_ids[name],
              ref.sample_ids[name], ref.gains[name])
      refcpu.sparse_dense_matmul(*args, table, bs, num_sc_per_device=1,
                                 num_scs=1, threads=threads)
      refcpu.sparse_dense_matmul_grad(*args, grad, table, acc,
                                      learning_rate=lr, num_sc_per_device=1,
                                      num_scs=1, threads=threads, inplace=True)
    busy += time.perf_counter() - t0
    iters += 1
  return {
      "value": total_lookups * iters / busy,
      "unit": "lookups/s",
      "cores": threads,
      "host_cpus": os.cpu_count(),
      "usable_cpus": _usable_cpus(),
      "cpu_model": _cpu_model(),
      "kind": "port",
      "sample": (f"first {sample_batch} samples of each of the "
                 f"{len(feats)} features ({total_lookups} lookups), "
                 f"{iters} fwd+bwd+optimizer passes in {busy:.1f} s; oracle "
                 f"preprocessing of the sample {pre_s * 1e3:.1f} ms on 1 "
                 "thread"),
      "preprocess_ms_per_1k_lookups": pre_s * 1e3 / total_lookups * 1e3,
      # The oracle's minibatching passes on the same sample (1 thread).
      "minibatching_preprocess_ms_per_1k_lookups": (
          mb[0] * 1e3 / total_lookups * 1e3 if mb else None),
      "minibatching_sample": (
          f"limit {mb[2]} ids per partition, {mb[1]} minibatches"
          if mb else None),
  }


CPU_SHARE = 16  # host cores a one-GPU job may use on the GPU boxes


def _usable_cpus() -> int:
  try:
    return len(os.sched_getaffinity(0))
  except (AttributeError, OSError):
    return os.cpu_count() or 1


def _cpu_model() -> str | None:
  try:
    with open("/proc/cpuinfo") as f:
      for line in f:
        if line.startswith("model name"):
          return line.split(":", 1)[1].strip()
  except OSError:
    pass
  return None


KERNEL_SOURCES = ("segreduce.h", "lookup.hip")


def kernel_sources_sha256() -> str:
  """SHA-256 over the sources of the measured kernels (the SegReduce /
  SegFinish templates and their launches), in KERNEL_SOURCES order."""
  import hashlib  # pylint: disable=g-import-not-at-top

  h = hashlib.sha256()
  for name in KERNEL_SOURCES:
    with open(os.path.join(ROOT, "jax-tpu-embedding_amd", "csrc", name),
              "rb") as f:
      h.update(f.read())
  return h.hexdigest()


def profiled_traffic():
  """HBM bytes per launch pair from the committed rocprofv3 --pmc summary,
  if it was measured on the current kernel sources (the summary names their
  SHA-256); else None."""
  import re  # pylint: disable=g-import-not-at-top

  summary = os.path.join(ROOT, "profiles", "dlrm26_segreduce_hbm_traffic.md")
  try:
    sha = kernel_sources_sha256()
    with open(summary) as f:
      text = f.read()
  except OSError:
    return None
  m = re.search(r"bench-traffic: kernel_sources_sha256=(\w+) bwd_bytes=(\d+) "
                r"fwd_bytes=(\d+)", text)
  if not m or m.group(1) != sha:
    return None
  return {"bwd": int(m.group(2)), "fwd": int(m.group(3))}


def main():
  ap = argparse.ArgumentParser()
  ap.add_argument("--gpus", type=int, default=1)
  ap.add_argument("--steps", type=int, default=20)
  ap.add_argument("--warmup", type=int, default=5)
  ap.add_argument("--cpu-seconds", type=float, default=10.0)
  ap.add_argument("--cpu-sample-batch", type=int, default=8192)
  ap.add_argument("--no-cpu-baseline", action="store_true")
  ap.add_argument("--copy-probe", action="store_true",
                  help="run a 1 GiB device copy first (counter calibration)")
  ap.add_argument("--no-api-steps", action="store_true",
                  help="skip timing the step through the embedding API")
  ap.add_argument("--no-optimizer-steps", action="store_true",
                  help="skip timing the backward with the other optimizers")
  ap.add_argument("--no-minibatching", action="store_true",
                  help="skip the minibatching leg (headline stack only)")
  ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS),
                  help="BASELINE.json config (c2, the 26-table DLRM shape, "
                       "is the headline)")
  args = ap.parse_args()
  if args.gpus != 1:
    print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
          "(this build has no multi-GPU path).", file=sys.stderr)
    sys.exit(2)
  t_setup = time.perf_counter()
  w = WORKLOADS[args.workload]()
  log(f"workload built in {time.perf_counter() - t_setup:.1f} s")
  res = run_gpu(w, args.steps, args.warmup, probe=args.copy_probe,
                api=not args.no_api_steps,
                # The headline stack only (two more table-sized slots do not
                # fit next to config 4's 205 GB table and accumulator).
                other_optimizers=(not args.no_optimizer_steps and
                                  w.name == "dlrm26"),
                minibatching=not args.no_minibatching and w.name == "dlrm26")
  fwd_bytes, bwd_bytes = algorithmic_bytes(res["per_stack"])
  step_s = res["ms_per_step"] / 1e3
  sp = res["spans"]
  # Each op is one SegReduce launch plus one SegFinish launch (the finish
  # kernel completes the rows whose entries span several blocks); the
  # backward adds its hot-run launches where they run (0 otherwise).
  fwd_ms = sp["fwd_reduce"][0] + sp["fwd_finish"][0]
  hot_ms = sp["bwd_hot_plan"][0] + sp["bwd_hot_reduce"][0]
  bwd_ms = sp["bwd_reduce"][0] + sp["bwd_finish"][0] + hot_ms
  traffic = profiled_traffic() if w.name == "dlrm26" else None
  opts = sorted({s["optimizer"] for s in res["per_stack"].values()})
  if bwd_ms >= fwd_ms:
    hot = " + hot runs" if hot_ms > 0 else ""
    dom, dom_ms, dom_bytes = (
        f"bwd: SegReduce+SegFinish{hot} ({'/'.join(opts)})", bwd_ms,
        bwd_bytes)
    dom_traffic = traffic["bwd"] if traffic else None
  else:
    dom, dom_ms, dom_bytes = "fwd: SegReduce+SegFinish", fwd_ms, fwd_bytes
    dom_traffic = traffic["fwd"] if traffic else None
  achieved = dom_bytes / (dom_ms / 1e3) / 1e9
  roofline = {
      "bound": "hbm",
      "kernel": dom,
      "achieved": round(achieved, 1),
      "peak": PEAK_HBM_GBS,
      "unit": "GB/s",
      "frac": round(achieved / PEAK_HBM_GBS, 4),
      # HBM bytes per launch pair, rocprofv3 FETCH_SIZE + WRITE_SIZE scaled
      # by a 1 GiB copy (profiles/dlrm26_segreduce_hbm_traffic.md).
      "traffic": dom_traffic,
      "kernel_ms": round(dom_ms, 4),
      "algorithmic_bytes": int(dom_bytes),
      # The same rate against a 1 GiB device copy timed in this run.
      "copy_gbs": round(res["copy_gbs"], 1),
      "copy_frac": round(achieved / res["copy_gbs"], 4),
  }
  cpu = None
  if not args.no_cpu_baseline:
    cpu = cpu_baseline(w, args.cpu_sample_batch, args.cpu_seconds,
                       minibatching=res["minibatching"] is not None)
  spans = {k: round(v[0], 4) for k, v in res["spans"].items()}
  out = {
      "metric": METRIC if w.name == "dlrm26" else METRIC.replace(
          "Adagrad), 26-table DLRM shape", "optimizer)"),
      "value": round(res["lookups"] / step_s, 1),
      "unit": "lookups/s",
      "n_gpus": 1,
      "steps": args.steps,
      "warmup": args.warmup,
      # Steps rotate through `num_batches` seeded batches (distinct ids,
      # CSRs and upstream gradients); the same step repeated on the first
      # batch, whose rows the caches then still hold, is beside it.
      "ms_per_step": round(res["ms_per_step"], 4),
      "num_batches": res["num_batches"],
      "same_batch_ms_per_step": round(res["same_batch_ms_per_step"], 4),
      "csr_only_ms_per_step": round(res["csr_only_ms_per_step"], 4),
      # The step replayed from a HIP graph (no per-call host work).
      "graph_ms_per_step": round(res["graph_ms_per_step"], 4),
      # Steady state with the next batch preprocessed on a second stream
      # while the step runs (preprocessing included, overlapped).
      "pipelined_ms_per_step": round(res["pipelined_ms_per_step"], 4),
      # The same step through the embedding API with per-feature tensors:
      # stacking fused into the kernels, and with unstack / stack copies.
      "api_ms_per_step": (round(res["api_ms_per_step"], 4)
                          if res["api_ms_per_step"] else None),
      "api_copy_ms_per_step": (round(res["api_copy_ms_per_step"], 4)
                               if res["api_copy_ms_per_step"] else None),
      "higher_is_better": True,
      "scaling": "weak",
      "vs_baseline": None,
      "dtype": "f32",
      "data": (f"synthetic ({res['num_batches']} seeded numpy batches of "
               "ids and N(0,1) grads in turn, N(0,0.01) tables)"),
      "config": w.description,
      "achieved_step_hbm_gbs": round((fwd_bytes + bwd_bytes) / step_s / 1e9,
                                     1),
      "step_hbm_frac": round((fwd_bytes + bwd_bytes) / step_s / 1e9 /
                             PEAK_HBM_GBS, 4),
      "step_copy_frac": round((fwd_bytes + bwd_bytes) / step_s / 1e9 /
                              res["copy_gbs"], 4),
      "algorithmic_bytes_per_step": int(fwd_bytes + bwd_bytes),
      # HIP-event time per step of each kernel (summed over stacks).
      "kernel_ms_per_step": spans,
      "preprocess_ms": round(res["preprocess_ms"], 3),
      "csr": res["per_stack"],
      "roofline": roofline,
      "cpu_baseline": cpu,
  }
  if res["optimizer_bwd_ms"]:
    # The same backward with each optimizer: compulsory bytes 12N + 4D*Bs +
    # 8D*U per table or slot array read and written.
    (s,) = res["per_stack"].values()

    def optimizer_bwd_bytes(slots):
      return (12 * s["N"] + 4 * s["D"] * s["Bs"] +
              8 * (1 + slots) * s["D"] * s["U"])

    out["optimizer_bwd"] = {
        k: {"ms": round(v, 4),
            "hbm_frac": round(
                optimizer_bwd_bytes(1 if k in ONE_SLOT_OPTIMIZERS else 2) /
                (v / 1e3) / 1e9 / PEAK_HBM_GBS, 4)}
        for k, v in res["optimizer_bwd_ms"].items()}
  if res["minibatching"]:
    # Same entries (nothing dropped), so the same compulsory bytes.
    mb = res["minibatching"]
    out["minibatching"] = {
        "num_minibatches": mb["num_minibatches"],
        "max_ids_per_partition": mb["max_ids_per_partition"],
        "preprocess_ms": round(mb["preprocess_ms"], 3),
        "ms_per_step": round(mb["ms_per_step"], 4),
        "step_hbm_frac": round((fwd_bytes + bwd_bytes) /
                               (mb["ms_per_step"] / 1e3) / 1e9 /
                               PEAK_HBM_GBS, 4),
        "dropped": mb["dropped"],
    }
  print(json.dumps(out), flush=True)


if __name__ == "__main__":
  main()
