"""Grouping a CSR by activation row (the CSR-only forward's sample stream).

The stream must be the stable sort of the CSR's valid entries by activation
row: each row's entries in CSR order, the order in which the oracle sums.
Activation rows of 9 to 21 key bits take one radix pass on the top 8 bits
and a sort of each of its 256 buckets by the low bits in one block (LDS
passes over chunks of 8,192 entries); wider keys take the LSD passes. The
cases below cover low-bit widths of 1 to 13 (one and two LDS passes),
buckets of one chunk and of several (a long row, and c3-sized buckets of
about 15,600 entries), rows of thousands of entries, empty buckets, padding
and alignment gaps, entries outside the table, and four segments.
Expectations come from numpy's stable argsort of the same CSR.
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
from jax_tpu_embedding.sparsecore.lib.core.primitives import _device  # pylint: disable=g-import-not-at-top,wrong-import-position

PAD = np.iinfo(np.int32).max


def _csr(rng, num_sc, bps, rpp, entries, heavy=0, bad=0.0, tail=0,
         unique=False, repeat=False):
  """A CSR of `num_sc` segments with `num_sc` partitions each: partition
  entries ascending by id, 8-aligned starts, padding to the segment end.
  `heavy` entries go to sample 3 of every segment (one long row). `tail`:
  that many more positions at the end of each segment, filled with entries
  that look valid (ids and samples in range) but lie past the last
  partition's row pointer, where the format leaves memory unwritten.
  `unique`: every activation row at most once per segment (one-hot rows);
  `repeat` then gives one row a second entry."""
  parts = num_sc
  per_part = entries // (num_sc * parts)
  per_seg = (parts * ((per_part + heavy // parts + 7) // 8 * 8) + 64 + tail)
  eid = np.full(num_sc * per_seg, PAD, np.int32)
  sid = np.full(num_sc * per_seg, PAD, np.int32)
  gains = np.full(num_sc * per_seg, np.nan, np.float32)
  rp = np.zeros((num_sc, parts), np.int32)
  for s in range(num_sc):
    start = 0
    perm = rng.permutation(bps).astype(np.int32) if unique else None
    for p in range(parts):
      c = per_part + heavy // parts
      ids = np.sort(rng.integers(0, rpp, size=c)).astype(np.int32)
      if bad:
        ids[rng.random(c) < bad] = rpp + 5
      if unique:
        rows = perm[p * c:(p + 1) * c].copy()
        if repeat and p == 0:
          rows[1] = rows[0]
      else:
        rows = rng.integers(0, bps, size=c).astype(np.int32)
      if heavy:
        rows[rng.permutation(c)[:heavy // parts]] = 3
      o = s * per_seg + start
      eid[o:o + c] = ids
      sid[o:o + c] = rows
      gains[o:o + c] = rng.uniform(0.5, 1.5, size=c).astype(np.float32)
      rp[s, p] = start + c
      start = (start + c + 7) // 8 * 8
    if tail:
      o, e = s * per_seg + start, (s + 1) * per_seg
      eid[o:e] = rng.integers(0, rpp, size=e - o)
      sid[o:e] = rng.integers(0, bps, size=e - o)
      gains[o:e] = 1.0
  return rp.reshape(-1), eid, sid, gains, per_seg


def _expected(rp, eid, sid, gains, num_sc, bps, rpp, per_seg):
  parts = rp.size // num_sc
  keys, ents = [], []
  g = gains.view(np.uint32).astype(np.uint64)
  for s in range(num_sc):
    start = 0
    for p in range(parts):
      end = int(rp[s * parts + p])
      sl = slice(s * per_seg + start, s * per_seg + end)
      e, r = eid[sl], sid[sl]
      ok = (e >= 0) & (e < rpp) & (r >= 0) & (r < bps)
      keys.append((s * bps + r[ok]).astype(np.int64))
      ents.append((p * rpp + e[ok]).astype(np.uint64) | (g[sl][ok] <<
                                                          np.uint64(32)))
      start = (end + 7) // 8 * 8
  keys = np.concatenate(keys)
  ents = np.concatenate(ents)
  order = np.argsort(keys, kind="stable")
  return keys[order], ents[order]


def _check(rng, num_sc, batch, entries, heavy=0, bad=0.0, tail=0,
           unique=False, repeat=False):
  bps = batch // num_sc
  rpp = 5000
  rp, eid, sid, gains, per_seg = _csr(rng, num_sc, bps, rpp, entries, heavy,
                                      bad, tail, unique, repeat)
  keep, c = _device.csr_operands(rp, eid, sid, gains, num_sc, num_sc)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  v = _native.build_sample_view(c, batch, rpp * num_sc, device_status=status)
  torch.cuda.synchronize()
  del keep
  ek, ee = _expected(rp, eid, sid, gains, num_sc, bps, rpp, per_seg)
  gk = v.keys.cpu().numpy().astype(np.int64)
  ge = v.entries.cpu().numpy().view(np.uint64)
  total = ek.size
  np.testing.assert_array_equal(gk[:total], ek)
  np.testing.assert_array_equal(ge[:total], ee)
  assert (gk[total:] == batch).all()
  st = int(status.item())
  assert bool(st & _native.STATUS_BAD_ENTRY) == bool(bad), st


# (batch, entries): keys of 9-13 bits (1-5 low bits: one LDS pass), 15, 17
# (also with buckets of two chunks), 19, 20 and 21 bits (7-13 low bits: two
# LDS passes), then 22 bits (LSD passes).
@pytest.mark.parametrize("batch,entries", [
    (300, 2000), (1000, 900), (2048, 30000), (4000, 20000), (8192, 8192),
    (20000, 100000), (100000, 400000), (70000, 4000000), (500000, 300000),
    (1 << 20, 300000), (1703936, 1703936), (2500000, 600000)])
def test_stream_is_the_stable_row_sort(batch, entries):
  _check(np.random.default_rng(batch), 1, batch, entries)


@pytest.mark.parametrize("repeat", [False, True])
@pytest.mark.parametrize("batch,entries", [
    (1000, 900), (8192, 8192), (500000, 300000), (1703936, 1703936)])
def test_rows_of_one_entry(batch, entries, repeat):
  """At most one entry per activation row: the buckets place entries by key
  without ranking. One repeated row sends its bucket back to the ranked
  passes (the others are still placed), with the same stream."""
  _check(np.random.default_rng(batch + 5), 1, batch, entries, unique=True,
         repeat=repeat)


@pytest.mark.parametrize("batch", [4000, 70000, 1703936])
def test_long_row_spans_several_bucket_chunks(batch):
  """Row 3 holds 150,000 entries: its bucket is sorted in 19 chunks."""
  _check(np.random.default_rng(batch + 1), 1, batch, 50000, heavy=150000)


@pytest.mark.parametrize("batch", [512, 131072])
def test_four_segments_and_entries_outside_the_table(batch):
  _check(np.random.default_rng(batch + 2), 4, batch, 80000, bad=0.05)


@pytest.mark.parametrize("batch,num_sc", [(20000, 1), (2500000, 1),
                                           (131072, 4)])
def test_entries_past_the_last_row_pointer_are_ignored(batch, num_sc):
  """Positions past each segment's last partition hold valid-looking
  entries (a buffer sized for more ids than the batch has, its end never
  written): the stream takes none of them, through the bucket route
  (batch 20,000), the LSD passes (2.5M rows) and four segments."""
  _check(np.random.default_rng(batch + 3), num_sc, batch, 60000, tail=40000)


@pytest.mark.parametrize("batch", [5000, 2500000])
def test_decreasing_row_pointers_forward_and_backward_agree(batch):
  """Row pointers that decrease (one segment, four partitions: 1600, 800,
  3200, 2400). A position belongs to the first partition whose row pointer
  lies past it, unless it falls in that partition's alignment gap, so the
  entries are positions [0, 1600) (partition 0) and [1600, 3200)
  (partition 2), and [3200, 4096) is padding. The CSR-only forward bounds
  its passes by the largest row pointer, not the last: it must take the
  same entries as the backward, which walks every position. Integer tables,
  gains and gradients make both sums exact, so the forward and the SGD
  update are compared bit for bit with numpy over those entries, through
  the bucket route (batch 5,000) and the LSD passes (2.5M rows)."""
  rng = np.random.default_rng(batch + 4)
  parts, rpp, dim, per_seg = 4, 3000, 8, 4096
  rp = np.array([1600, 800, 3200, 2400], np.int32)
  eid = np.sort(rng.integers(0, rpp, size=per_seg)).astype(np.int32)
  eid[1600:3200] = np.sort(rng.integers(0, rpp, size=1600))
  sid = rng.integers(0, batch, size=per_seg).astype(np.int32)
  gains = rng.integers(1, 4, size=per_seg).astype(np.float32)
  table = rng.integers(-8, 9, size=(parts * rpp, dim)).astype(np.float32)
  grad = rng.integers(-4, 5, size=(batch, dim)).astype(np.float32)
  part = np.full(per_seg, -1)
  part[:1600] = 0
  part[1600:3200] = 2
  ok = part >= 0
  rows = part[ok] * rpp + eid[ok]
  exp_act = np.zeros((batch, dim), np.float64)
  np.add.at(exp_act, sid[ok], gains[ok, None] * table[rows])
  exp_table = table.astype(np.float64)
  np.add.at(exp_table, rows, -gains[ok, None] * grad[sid[ok]])
  keep, c = _device.csr_operands(rp, eid, sid, gains, 1, parts)
  status = torch.zeros(1, dtype=torch.int32, device="cuda")
  table_t = torch.from_numpy(table).cuda()
  act = torch.zeros((batch, dim), dtype=torch.float32, device="cuda")
  _native.sparse_dense_matmul(c, table_t, act, batch, device_status=status)
  _native.sparse_dense_matmul_grad(c, torch.from_numpy(grad).cuda(), table_t,
                                   None, 1.0, batch, device_status=status)
  torch.cuda.synchronize()
  del keep
  assert int(status.item()) == 0
  np.testing.assert_array_equal(act.cpu().numpy(), exp_act.astype(np.float32))
  np.testing.assert_array_equal(table_t.cpu().numpy(),
                                exp_table.astype(np.float32))
