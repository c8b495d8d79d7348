"""ctypes binding of libscemb.so (the C ABI declared in include/scemb.h).

This is the only place where Python touches the native library. Device memory
and streams come from torch: tensors are passed by ``data_ptr()`` and kernels
are enqueued on ``torch.cuda.current_stream()``. There is no fallback: if the
library or a GPU is missing, calls raise.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import struct
import threading

import numpy as np

_PKG_ROOT = pathlib.Path(__file__).resolve().parents[2]
LIB_PATH = pathlib.Path(
    os.environ.get("SCEMB_LIBRARY", str(_PKG_ROOT / "libscemb.so")))

SCEMB_OK = 0
SCEMB_ERR_INVALID_ARGUMENT = 1
SCEMB_ERR_NOT_IMPLEMENTED = 2
SCEMB_ERR_WORKSPACE = 3
SCEMB_ERR_DEVICE = 4
SCEMB_ERR_LIMIT_EXCEEDED = 5

STATUS_BAD_ENTRY = 1
STATUS_BAD_ID = 2
STATUS_UNSORTED = 4
STATUS_SHARED_ROW = 8

CSR_SORTED_BY_ROW = 1
CSR_ONE_ENTRY_PER_ROW = 2

# scemb_optimizer_t kinds and flags.
OPTIMIZER_SGD = 0
OPTIMIZER_ADAGRAD = 1
OPTIMIZER_ADAM = 2
OPTIMIZER_ADAGRAD_MOMENTUM = 3
OPTIMIZER_FTRL = 4
OPTIMIZER_LAPROP = 5
OPTIMIZER_F2A = 6
OPTIMIZER_CUSTOM = 7
MAX_HYPERPARAMETERS = 8
PROGRAM_MAX_OPS = 48
OPTIMIZER_FLAG_MULTIPLY_LINEAR_BY_LR = 1

# Every function declared in include/scemb.h.
EXPORTED_SYMBOLS = (
    "scemb_last_error",
    "scemb_version",
    "scemb_sparse_dense_matmul_workspace_size",
    "scemb_sparse_dense_matmul",
    "scemb_sparse_dense_matmul_no_alloc",
    "scemb_sparse_dense_matmul_to_blocks",
    "scemb_activation_unstack",
    "scemb_gradient_stack",
    "scemb_build_sample_view_workspace_size",
    "scemb_build_sample_view",
    "scemb_sparse_dense_matmul_grad_workspace_size",
    "scemb_sparse_dense_matmul_grad_with_sgd",
    "scemb_sparse_dense_matmul_grad_with_adagrad",
    "scemb_sparse_dense_matmul_grad_with_sgd_from_blocks",
    "scemb_sparse_dense_matmul_grad_with_adagrad_from_blocks",
    "scemb_sparse_dense_matmul_grad_with_optimizer",
    "scemb_sparse_dense_matmul_grad_with_optimizer_from_blocks",
    "scemb_preprocess_stats_size",
    "scemb_preprocess_stats_counters_offset",
    "scemb_preprocess_workspace_size",
    "scemb_preprocess_stacked_table",
    "scemb_preprocess_stacked_tables",
    "scemb_check_row_splits",
    "scemb_stage_row_splits",
    "scemb_stage_row_splits_batch",
    "scemb_compute_theoretical_max_coo_buffer_size",
    "scemb_compute_coo_buffer_size_per_device",
    "scemb_compute_row_pointers_size_per_device",
    "scemb_profile_enable",
    "scemb_profile_collect",
)


class Csr(ctypes.Structure):
  _fields_ = [
      ("row_pointers", ctypes.c_void_p),
      ("embedding_ids", ctypes.c_void_p),
      ("sample_ids", ctypes.c_void_p),
      ("gains", ctypes.c_void_p),
      ("coo_size", ctypes.c_int64),
      ("num_segments", ctypes.c_int32),
      ("num_partitions", ctypes.c_int32),
      ("row_pointers_per_segment", ctypes.c_int32),
      ("flags", ctypes.c_uint32),
      ("num_entries", ctypes.c_int64),
      ("num_minibatches", ctypes.c_int32),
      ("positions_used", ctypes.c_int32),
  ]


class SampleView(ctypes.Structure):
  _fields_ = [
      ("keys", ctypes.c_void_p),
      ("entries", ctypes.c_void_p),
      ("size", ctypes.c_int64),
      ("device_batch_size", ctypes.c_int64),
      ("table_rows", ctypes.c_int64),
      ("num_entries", ctypes.c_int64),
      ("flags", ctypes.c_uint32),
      ("reserved", ctypes.c_int32),
  ]


VIEW_ONE_ENTRY_PER_KEY = 1


class RowBlock(ctypes.Structure):
  _fields_ = [
      ("first_row", ctypes.c_int64),
      ("num_rows", ctypes.c_int64),
      ("data", ctypes.c_void_p),
      ("row_stride", ctypes.c_int64),
      ("width", ctypes.c_int32),
      ("reserved", ctypes.c_int32),
  ]


MAX_ROW_BLOCKS = 32
# Minibatching buckets per SparseCore, the most minibatches (coo_format.h:
# 52-53).
MAX_MINIBATCHES = 64


class UpdateProgram(ctypes.Structure):
  _fields_ = [
      ("num_ops", ctypes.c_int32),
      ("num_slots", ctypes.c_int32),
      ("num_hyperparameters", ctypes.c_int32),
      ("op", ctypes.c_uint8 * PROGRAM_MAX_OPS),
      ("dst", ctypes.c_uint8 * PROGRAM_MAX_OPS),
      ("a", ctypes.c_uint8 * PROGRAM_MAX_OPS),
      ("b", ctypes.c_uint8 * PROGRAM_MAX_OPS),
      ("c", ctypes.c_uint8 * PROGRAM_MAX_OPS),
      ("imm", ctypes.c_float * PROGRAM_MAX_OPS),
      ("out", ctypes.c_uint8 * 3),
      ("reserved", ctypes.c_uint8),
  ]


def update_program(fields: dict) -> UpdateProgram:
  """scemb_update_program_t from UpdateProgram.compile()'s fields."""
  p = UpdateProgram()
  p.num_ops = len(fields["op"])
  p.num_slots = fields["num_slots"]
  p.num_hyperparameters = fields["num_hyperparameters"]
  for k in ("op", "dst", "a", "b", "c", "imm"):
    arr = getattr(p, k)
    for i, v in enumerate(fields[k]):
      arr[i] = v
  for i, v in enumerate(fields["out"]):
    p.out[i] = v
  return p


class Optimizer(ctypes.Structure):
  _fields_ = [
      ("kind", ctypes.c_int32),
      ("flags", ctypes.c_uint32),
      ("slots", ctypes.c_void_p * 2),
      ("hyperparameter_ptrs", ctypes.c_void_p * MAX_HYPERPARAMETERS),
      ("hyperparameters", ctypes.c_float * MAX_HYPERPARAMETERS),
      ("clip_mask", ctypes.c_int32),
      ("min_value", ctypes.c_float),
      ("max_value", ctypes.c_float),
      ("program", ctypes.POINTER(UpdateProgram)),
  ]


class Feature(ctypes.Structure):
  _fields_ = [
      ("ids", ctypes.c_void_p),
      ("weights", ctypes.c_void_p),
      ("row_splits", ctypes.c_void_p),
      ("row_splits_host", ctypes.c_void_p),
      ("num_rows", ctypes.c_int64),
      ("nnz", ctypes.c_int64),
      ("valency", ctypes.c_int32),
      ("row_offset", ctypes.c_int32),
      ("col_offset", ctypes.c_int32),
      ("col_shift", ctypes.c_int32),
      ("max_row_length", ctypes.c_int64),
  ]


# scemb_feature_t packed by one precompiled struct: four addresses, two
# int64, four int32, one int64, with no padding (checked below). Packing the
# rows is several times cheaper than building a ctypes structure or a numpy
# record per feature.
_FEATURE_STRUCT = struct.Struct("<QQQQqqiiiiq")
assert _FEATURE_STRUCT.size == ctypes.sizeof(Feature) and [
    getattr(Feature, f[0]).offset for f in Feature._fields_] == [
        0, 8, 16, 24, 32, 40, 48, 52, 56, 60, 64]


class FeatureArray:
  """scemb_feature_t[n] in a ctypes buffer; pass it where the C ABI takes
  the features (the array must outlive the call)."""

  def __init__(self, rows):
    pack = _FEATURE_STRUCT.pack
    data = b"".join([pack(r[0] or 0, r[1] or 0, r[2] or 0, r[3] or 0, *r[4:])
                     for r in rows])
    self._n = len(rows)
    self._buffer = ctypes.create_string_buffer(data, max(len(data), 1))
    self._as_parameter_ = ctypes.cast(self._buffer, ctypes.POINTER(Feature))

  def __len__(self):
    return self._n

  @property
  def address(self) -> int:
    return ctypes.addressof(self._buffer)


def feature_structs(rows) -> FeatureArray:
  """scemb_feature_t[len(rows)] from (ids, weights, row_splits,
  row_splits_host, num_rows, nnz, valency, row_offset, col_offset,
  col_shift, max_row_length) tuples; addresses may be None (null)."""
  return FeatureArray(rows)


class PreprocessOptions(ctypes.Structure):
  _fields_ = [
      ("local_device_count", ctypes.c_int32),
      ("global_device_count", ctypes.c_int32),
      ("num_sc_per_device", ctypes.c_int32),
      ("combiner", ctypes.c_int32),
      ("max_ids_per_partition", ctypes.c_int32),
      ("max_unique_ids_per_partition", ctypes.c_int32),
      ("allow_id_dropping", ctypes.c_int32),
      ("has_variable_weights", ctypes.c_int32),
      ("coo_buffer_size_per_device", ctypes.c_int64),
      ("col_id_bound", ctypes.c_int64),
      ("build_sample_view", ctypes.c_int32),
      ("enable_minibatching", ctypes.c_int32),
      ("table_rows", ctypes.c_int64),
      ("minibatching_pass", ctypes.c_int32),
      ("flags", ctypes.c_int32),
      ("minibatching_split", ctypes.c_uint64),
  ]


# PreprocessOptions.flags: merge duplicates after the sort even where the
# library would merge them at extraction (both give the same outputs).
PREPROCESS_GROUP_AFTER_SORT = 1


class PreprocessOutput(ctypes.Structure):
  _fields_ = [
      ("row_pointers", ctypes.c_void_p),
      ("embedding_ids", ctypes.c_void_p),
      ("sample_ids", ctypes.c_void_p),
      ("gains", ctypes.c_void_p),
      ("stats", ctypes.c_void_p),
      ("view_keys", ctypes.c_void_p),
      ("view_entries", ctypes.c_void_p),
  ]


class PreprocessJob(ctypes.Structure):
  """scemb_preprocess_job_t: one stack of scemb_preprocess_stacked_tables
  (addresses of its features, options and outputs, which the caller keeps
  alive through the call)."""
  _fields_ = [
      ("features", ctypes.c_void_p),
      ("num_features", ctypes.c_int32),
      ("options", ctypes.c_void_p),
      ("outputs", ctypes.c_void_p),
      ("workspace", ctypes.c_void_p),
      ("workspace_bytes", ctypes.c_size_t),
  ]


_lib = None
_lib_lock = threading.Lock()


def load_library() -> ctypes.CDLL:
  """Loads libscemb.so; raises RuntimeError when it was not built."""
  global _lib
  with _lib_lock:
    if _lib is not None:
      return _lib
    if not LIB_PATH.exists():
      raise RuntimeError(
          f"libscemb.so not found at {LIB_PATH}; build it with "
          "`python -c 'import __graft_entry__; __graft_entry__.build()'` or "
          "`make -C jax-tpu-embedding_amd/csrc`.")
    # torch first: its wheel carries its own HIP runtime, which libscemb's
    # libamdhip64 dependency must resolve to. Loaded the other way round, the
    # process holds two runtimes and launches from the library find no
    # device.
    import torch as _  # pylint: disable=g-import-not-at-top,unused-import
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, i32, i64, f32, sz = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                             ctypes.c_float, ctypes.c_size_t)
    csr_p = ctypes.POINTER(Csr)
    view_p = ctypes.POINTER(SampleView)
    lib.scemb_last_error.restype = ctypes.c_char_p
    lib.scemb_last_error.argtypes = []
    lib.scemb_version.restype = ctypes.c_int
    lib.scemb_version.argtypes = []
    lib.scemb_sparse_dense_matmul_workspace_size.restype = sz
    lib.scemb_sparse_dense_matmul_workspace_size.argtypes = [
        csr_p, view_p, i64, i64, i32]
    lib.scemb_sparse_dense_matmul.restype = ctypes.c_int
    lib.scemb_sparse_dense_matmul.argtypes = [csr_p, view_p, vp, i64, i32, vp,
                                              i64, vp, sz, vp, vp]
    lib.scemb_sparse_dense_matmul_no_alloc.restype = ctypes.c_int
    lib.scemb_sparse_dense_matmul_no_alloc.argtypes = [
        csr_p, view_p, vp, i64, i32, vp, i64, vp, vp]
    blk_p = ctypes.POINTER(RowBlock)
    lib.scemb_sparse_dense_matmul_to_blocks.restype = ctypes.c_int
    lib.scemb_sparse_dense_matmul_to_blocks.argtypes = [
        csr_p, view_p, vp, i64, i32, blk_p, i32, i64, vp, sz, vp, vp]
    lib.scemb_sparse_dense_matmul_grad_with_sgd_from_blocks.restype = (
        ctypes.c_int)
    lib.scemb_sparse_dense_matmul_grad_with_sgd_from_blocks.argtypes = [
        csr_p, blk_p, i32, i64, vp, i64, i32, vp, f32, i32, f32, f32, vp, sz,
        vp, vp]
    lib.scemb_sparse_dense_matmul_grad_with_adagrad_from_blocks.restype = (
        ctypes.c_int)
    lib.scemb_sparse_dense_matmul_grad_with_adagrad_from_blocks.argtypes = [
        csr_p, blk_p, i32, i64, vp, vp, i64, i32, vp, f32, i32, f32, f32, vp,
        sz, vp, vp]
    lib.scemb_activation_unstack.restype = ctypes.c_int
    lib.scemb_activation_unstack.argtypes = [vp, i64, i32, blk_p, i32, vp]
    lib.scemb_gradient_stack.restype = ctypes.c_int
    lib.scemb_gradient_stack.argtypes = [blk_p, i32, vp, i64, i32, vp]
    lib.scemb_build_sample_view_workspace_size.restype = sz
    lib.scemb_build_sample_view_workspace_size.argtypes = [csr_p, i64, i64]
    lib.scemb_build_sample_view.restype = ctypes.c_int
    lib.scemb_build_sample_view.argtypes = [csr_p, i64, i64, vp, vp, vp, sz,
                                            vp, vp]
    lib.scemb_sparse_dense_matmul_grad_workspace_size.restype = sz
    lib.scemb_sparse_dense_matmul_grad_workspace_size.argtypes = [
        csr_p, i64, i64, i32]
    lib.scemb_sparse_dense_matmul_grad_with_sgd.restype = ctypes.c_int
    lib.scemb_sparse_dense_matmul_grad_with_sgd.argtypes = [
        csr_p, vp, i64, vp, i64, i32, vp, f32, i32, f32, f32, vp, sz, vp, vp]
    lib.scemb_sparse_dense_matmul_grad_with_adagrad.restype = ctypes.c_int
    lib.scemb_sparse_dense_matmul_grad_with_adagrad.argtypes = [
        csr_p, vp, i64, vp, vp, i64, i32, vp, f32, i32, f32, f32, vp, sz, vp,
        vp]
    opt_p = ctypes.POINTER(Optimizer)
    lib.scemb_sparse_dense_matmul_grad_with_optimizer.restype = ctypes.c_int
    lib.scemb_sparse_dense_matmul_grad_with_optimizer.argtypes = [
        csr_p, vp, i64, vp, i64, i32, opt_p, vp, sz, vp, vp]
    lib.scemb_sparse_dense_matmul_grad_with_optimizer_from_blocks.restype = (
        ctypes.c_int)
    lib.scemb_sparse_dense_matmul_grad_with_optimizer_from_blocks.argtypes = [
        csr_p, blk_p, i32, i64, vp, i64, i32, opt_p, vp, sz, vp, vp]
    opts_p = ctypes.POINTER(PreprocessOptions)
    lib.scemb_preprocess_stats_size.restype = i64
    lib.scemb_preprocess_stats_size.argtypes = [opts_p]
    lib.scemb_preprocess_stats_counters_offset.restype = i64
    lib.scemb_preprocess_stats_counters_offset.argtypes = [opts_p]
    lib.scemb_preprocess_workspace_size.restype = sz
    lib.scemb_preprocess_workspace_size.argtypes = [ctypes.POINTER(Feature),
                                                    i32, opts_p]
    lib.scemb_preprocess_stacked_table.restype = ctypes.c_int
    lib.scemb_preprocess_stacked_table.argtypes = [
        ctypes.POINTER(Feature), i32, opts_p, ctypes.POINTER(PreprocessOutput),
        vp, sz, vp]
    lib.scemb_preprocess_stacked_tables.restype = ctypes.c_int
    lib.scemb_preprocess_stacked_tables.argtypes = [
        ctypes.POINTER(PreprocessJob), i32, vp]
    lib.scemb_check_row_splits.restype = ctypes.c_int
    lib.scemb_check_row_splits.argtypes = [vp, i64, i64,
                                           ctypes.POINTER(ctypes.c_int64)]
    lib.scemb_stage_row_splits.restype = ctypes.c_int
    lib.scemb_stage_row_splits.argtypes = [vp, i64, i64, vp,
                                           ctypes.POINTER(ctypes.c_int64)]
    lib.scemb_stage_row_splits_batch.restype = ctypes.c_int
    lib.scemb_stage_row_splits_batch.argtypes = [
        i32, vp, vp, vp, vp, vp, ctypes.POINTER(ctypes.c_int32)]
    lib.scemb_compute_theoretical_max_coo_buffer_size.restype = i64
    lib.scemb_compute_theoretical_max_coo_buffer_size.argtypes = [i32, i32,
                                                                  i32, i32]
    lib.scemb_compute_coo_buffer_size_per_device.restype = i64
    lib.scemb_compute_coo_buffer_size_per_device.argtypes = [i32, i64, i32,
                                                             i32, i32]
    lib.scemb_compute_row_pointers_size_per_device.restype = i32
    lib.scemb_compute_row_pointers_size_per_device.argtypes = [i32, i32, i32]
    lib.scemb_profile_enable.restype = None
    lib.scemb_profile_enable.argtypes = [ctypes.c_int]
    lib.scemb_profile_collect.restype = ctypes.c_int
    lib.scemb_profile_collect.argtypes = [ctypes.c_char_p,
                                          ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_int64)]
    _lib = lib
    return lib


def profile_enable(on: bool) -> None:
  """Turns the library's launch-timing events on or off."""
  load_library().scemb_profile_enable(1 if on else 0)


def profile_collect(name: str | None) -> tuple[float, int]:
  """(summed milliseconds, launches) of the spans recorded under `name`."""
  ms = ctypes.c_double(0.0)
  n = ctypes.c_int64(0)
  check(load_library().scemb_profile_collect(
      None if name is None else name.encode(), ctypes.byref(ms),
      ctypes.byref(n)))
  return ms.value, n.value


def check(rc: int) -> None:
  """Maps a libscemb status code to the reference's Python exceptions."""
  if rc == SCEMB_OK:
    return
  msg = load_library().scemb_last_error().decode("utf-8", "replace")
  if rc == SCEMB_ERR_INVALID_ARGUMENT:
    raise ValueError(msg)
  if rc == SCEMB_ERR_NOT_IMPLEMENTED:
    raise NotImplementedError(msg)
  raise RuntimeError(f"libscemb error {rc}: {msg}")


# Validation mode: the lookup and update primitives hand the kernels a
# device status word and read it back after each call (one host wait per
# call), raising on what the kernels found: entries out of range (skipped),
# or a stream declared sorted / with unrepeated keys that is not (results
# not valid). Off by default; SCEMB_VALIDATE=1 in the environment or
# set_validation(True) turns it on.
_validate = os.environ.get("SCEMB_VALIDATE", "0") not in ("", "0")

_STATUS_NAMES = (
    (STATUS_BAD_ENTRY, "CSR entry with an embedding or sample id out of "
     "range (skipped)"),
    (STATUS_BAD_ID, "input id outside the table (skipped)"),
    (STATUS_UNSORTED, "a stream declared sorted is not (results not valid)"),
    (STATUS_SHARED_ROW, "a stream declared with one entry per row repeats a "
     "row (results not valid)"),
)


def set_validation(on: bool) -> bool:
  """Turns validation mode on or off; returns the previous setting."""
  global _validate
  prev, _validate = _validate, bool(on)
  return prev


def validation() -> bool:
  return _validate


def status_word():
  """A zeroed device status word in validation mode, else None."""
  if not _validate:
    return None
  t = torch()
  return t.zeros(1, dtype=t.int32, device=device())


def raise_on_status(flags: int, what: str) -> None:
  """RuntimeError naming every status bit set in `flags`."""
  flags = int(flags) & 0xFFFFFFFF
  if flags == 0:
    return
  found = [text for bit, text in _STATUS_NAMES if flags & bit]
  raise RuntimeError(f"{what}: device status {flags:#x}: " + "; ".join(found))


def check_status_word(word, what: str) -> None:
  """Waits for the stream and raises on a non-zero status word (None: no
  check)."""
  if word is not None:
    raise_on_status(int(word.item()), what)


# ---------------------------------------------------------------------------
# torch plumbing.
# ---------------------------------------------------------------------------


def torch():
  import torch as _torch  # pylint: disable=g-import-not-at-top

  return _torch


_gpu_seen = False


def require_gpu():
  """torch, once a GPU has been seen (the check is not repeated: it costs
  more host time than a kernel launch)."""
  global _gpu_seen
  t = torch()
  if not _gpu_seen:
    if not t.cuda.is_available():
      raise RuntimeError(
          "The SparseCore embedding path runs on the GPU through "
          "libscemb.so; no GPU is visible to torch.")
    _gpu_seen = True
  return t


# Side streams for independent work within one call: a pool per (device,
# calling stream), created on first use, default priority. Calls made from
# different streams therefore never queue behind each other's side work nor
# share its workspaces (one per stream, below). Three side streams plus the
# calling stream match the four hardware queues a process gets by default.
NUM_SIDE_STREAMS = 3
_side_streams = {}


_hip = None


def _new_stream(dev: int):
  """A HIP stream of its own (non-blocking, default priority), wrapped for
  torch. torch.cuda.Stream() hands out a fixed pool of streams round robin,
  so two pools built from it can share a stream, and a side stream can be
  the very stream another caller uses; these are never shared. They live
  until the process ends."""
  global _hip
  t = torch()
  if _hip is None:
    # The HIP runtime torch runs on (its own copy when it ships one), so
    # that the stream belongs to the same runtime instance.
    own = pathlib.Path(t.__file__).parent / "lib" / "libamdhip64.so"
    _hip = ctypes.CDLL(str(own) if own.exists() else "libamdhip64.so")
    _hip.hipStreamCreateWithFlags.argtypes = [
        ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
    _hip.hipStreamCreateWithFlags.restype = ctypes.c_int
  with t.cuda.device(dev):
    h = ctypes.c_void_p()
    rc = _hip.hipStreamCreateWithFlags(ctypes.byref(h), 1)  # NonBlocking
    if rc != 0:
      raise RuntimeError(f"hipStreamCreateWithFlags failed ({rc})")
    return t.cuda.ExternalStream(h.value, device=dev)


def side_streams(n: int) -> list:
  """The first n side streams of the current device's current stream."""
  if n <= 0:
    return []
  t = torch()
  dev = t.cuda.current_device()
  key = (dev, t.cuda.current_stream(dev).cuda_stream)
  pool = _side_streams.get(key)
  if pool is None or len(pool) < n:
    pool = (pool or []) + [
        _new_stream(dev)
        for _ in range(max(n, NUM_SIDE_STREAMS) - len(pool or []))]
    _side_streams[key] = pool
  return pool[:n]


def _tensors_in(obj, out):
  t = torch()
  if isinstance(obj, t.Tensor):
    out.append(obj)
  elif isinstance(obj, dict):
    for v in obj.values():
      _tensors_in(v, out)
  elif isinstance(obj, (list, tuple)):
    for v in obj:
      _tensors_in(v, out)
  elif hasattr(obj, "__dict__"):
    for v in vars(obj).values():
      _tensors_in(v, out)
  return out


def run_per_stack(names, fn, width=None) -> dict:
  """{name: fn(name)} for independent per-stack calls (their own tables,
  inputs and outputs). Stacks of different widths (width(name), e.g. the
  embedding dimension) run concurrently, each width on its own side stream
  of the current stream (round robin): the narrow stacks' latency-bound
  kernels then fill the gaps and tails of the wide stacks' bandwidth-bound
  ones. Stacks of one width run one after another on their stream, as
  concurrent copies of the same bandwidth-bound kernel only compete for the
  same L2 and HBM. The current stream then waits for all of them; results
  allocated on a side stream are marked as used by the current stream, so
  their memory is not recycled before the caller's later work. A single
  width, no side streams (NUM_SIDE_STREAMS = 0) or no GPU: inline."""
  names = list(names)
  t = torch()
  widths = [width(n) if width else n for n in names]
  distinct = list(dict.fromkeys(widths))
  if (len(distinct) <= 1 or NUM_SIDE_STREAMS <= 0 or
      not t.cuda.is_available()):
    return {n: fn(n) for n in names}
  main = t.cuda.current_stream()
  sides = side_streams(min(len(distinct), NUM_SIDE_STREAMS))
  for s in sides:
    s.wait_stream(main)
  out = {}
  for n, w in zip(names, widths):
    with t.cuda.stream(sides[distinct.index(w) % len(sides)]):
      out[n] = fn(n)
  for s in sides:
    main.wait_stream(s)
  if not t.cuda.is_current_stream_capturing():
    for x in _tensors_in(out, []):
      if x.is_cuda:
        x.record_stream(main)
  return out


def stream_handle() -> int:
  t = torch()
  return t.cuda.current_stream().cuda_stream


def device() -> "torch.device":
  t = require_gpu()
  return t.device("cuda", t.cuda.current_device())


def as_device_tensor(x, dtype, dev=None):
  """Returns x as a contiguous CUDA tensor of `dtype` (copies if needed)."""
  t = require_gpu()
  dev = dev or device()
  if isinstance(x, t.Tensor):
    if x.device != dev or x.dtype != dtype:
      x = x.to(device=dev, dtype=dtype)
    return x.contiguous()
  arr = np.asarray(x)
  np_dtype = {t.int32: np.int32, t.int64: np.int64,
              t.float32: np.float32}[dtype]
  arr = np.ascontiguousarray(arr, dtype=np_dtype)
  return t.from_numpy(arr).to(dev, non_blocking=False)


ROW_SPLITS_MESSAGE = ("row_splits must start at 0, be non-decreasing and "
                      "end at the number of values.")


class HostUploads:
  """Host arrays bound for the device, gathered into one pinned staging
  buffer and sent with a single asynchronous copy on the current stream.

  add() returns a handle; after flush(), resolve(handle) is the device
  tensor (anything that is not a handle resolves to itself). The staging
  buffer comes from torch's pinned-memory cache, which keeps it until the
  copy has completed; nothing here waits for the device."""

  _ALIGN = 256  # every array starts 256-byte aligned on the device

  class _Handle:
    __slots__ = ("offset", "count", "dtype", "base", "nnz",
                 "max_row_length")

    def __init__(self, offset, count, dtype, nnz=None):
      self.offset, self.count, self.dtype = offset, count, dtype
      self.base = None  # the device buffer, after flush()
      self.nnz = nnz  # row splits: the number of values they end at
      self.max_row_length = None

    @property
    def tensor(self):
      if self.base is None:
        return None
      size = self.count * torch().empty(0, dtype=self.dtype).element_size()
      return self.base[self.offset:self.offset + size].view(self.dtype)

    @property
    def address(self):
      return None if self.base is None else self.base.data_ptr() + self.offset

  Handle = _Handle

  def __init__(self):
    self._items = []
    self._nbytes = 0

  def add(self, x, dtype, nnz=None):
    t = torch()
    np_dtype = {t.int32: np.int32, t.int64: np.int64,
                t.float32: np.float32}[dtype]
    arr = np.ascontiguousarray(np.asarray(x), dtype=np_dtype).reshape(-1)
    off = -(-self._nbytes // self._ALIGN) * self._ALIGN
    self._nbytes = off + arr.nbytes
    h = HostUploads._Handle(off, arr.size, dtype, nnz)
    self._items.append((arr, h))
    return h

  def add_row_splits(self, splits, nnz: int):
    """Host row splits of a ragged feature. flush() checks them
    (scemb_stage_row_splits: start at 0, non-decreasing, end at `nnz`) while
    it stages them, raising ValueError if they do not hold; the handle then
    holds their longest row in max_row_length."""
    if np.asarray(splits).size == 0:
      raise ValueError(ROW_SPLITS_MESSAGE)
    return self.add(splits, torch().int64, nnz)

  def flush(self):
    if not self._items:
      return
    t = torch()
    dev = device()
    host = t.empty(self._nbytes, dtype=t.uint8, pin_memory=True)
    staged = host.numpy()
    base = host.data_ptr()
    splits = []
    for arr, h in self._items:
      if h.nnz is None:
        staged[h.offset:h.offset + arr.nbytes] = arr.view(np.uint8)
      else:
        splits.append((arr, h))
    if splits:
      # Every feature's row splits checked and staged by one library call
      # (its rows spread over a few host threads).
      n = len(splits)
      src = np.fromiter((a.ctypes.data for a, _ in splits), np.uint64, n)
      rows = np.fromiter((a.size - 1 for a, _ in splits), np.int64, n)
      nnz = np.fromiter((h.nnz for _, h in splits), np.int64, n)
      dst = np.fromiter((base + h.offset for _, h in splits), np.uint64, n)
      longest = np.zeros(n, np.int64)
      bad = ctypes.c_int32(-1)
      if load_library().scemb_stage_row_splits_batch(
          n, src.ctypes.data, rows.ctypes.data, nnz.ctypes.data,
          dst.ctypes.data, longest.ctypes.data, ctypes.byref(bad)):
        self._items = []
        self._nbytes = 0
        raise ValueError(ROW_SPLITS_MESSAGE)
      for (_, h), most in zip(splits, longest.tolist()):
        h.max_row_length = most
    dst = t.empty(self._nbytes, dtype=t.uint8, device=dev)
    dst.copy_(host, non_blocking=True)
    for _, h in self._items:
      h.base = dst
    self._items = []
    self._nbytes = 0

  @staticmethod
  def resolve(x):
    """The device tensor of a handle; anything else as is."""
    if isinstance(x, HostUploads._Handle):
      if x.base is None:
        raise RuntimeError("HostUploads.flush() has not run")
      return x.tensor
    return x

  @staticmethod
  def resolve_address(x):
    """The device address of a handle (an int; its buffer stays alive while
    any tensor of the call holds it, see flush); anything else as is."""
    if isinstance(x, HostUploads._Handle):
      if x.base is None:
        raise RuntimeError("HostUploads.flush() has not run")
      return x.address
    return x


def ptr(x) -> int | None:
  """Device address of a tensor; an int address is passed through."""
  if x is None or isinstance(x, int):
    return x
  return x.data_ptr()


class _Workspace:
  """Scratch memory of the library's calls: one buffer per (device, stream),
  grown on demand and reused by later calls on the same stream, which stream
  order makes safe. Calls on different streams never share a buffer (the
  side streams a call forks to belong to its calling stream, see
  side_streams), so preprocessing on one stream may overlap a step or
  another preprocessing on another.

  A buffer that a call used while its stream was being captured into a graph
  stays allocated after it has been outgrown: the graph's replays still
  address it."""

  def __init__(self):
    self._buf = {}
    self._captured = set()
    self._retired = []

  def get(self, nbytes: int, stream=None):
    """The buffer of `stream` (default: the current stream), at least
    `nbytes` long. A new buffer is allocated on that stream, so that the
    allocator hands its memory to no other stream before the stream's work
    on it is done."""
    t = torch()
    dev = device()
    if stream is None:
      stream = t.cuda.current_stream(dev)
    key = (dev.index, stream.cuda_stream)
    buf = self._buf.get(key)
    if buf is None or buf.numel() < nbytes:
      if buf is not None and key in self._captured:
        self._retired.append(buf)
      with t.cuda.stream(stream):
        buf = t.empty(max(int(nbytes * 1.25), 1 << 20), dtype=t.uint8,
                      device=dev)
      self._buf[key] = buf
    if t.cuda.is_current_stream_capturing():
      self._captured.add(key)
    return buf


WORKSPACE = _Workspace()


def make_csr(row_pointers, embedding_ids, sample_ids, gains, num_segments,
             num_partitions, sorted_by_row: bool = False,
             num_entries: int | None = None,
             one_entry_per_row: bool = False,
             num_minibatches: int = 0, positions_used: int = 0) -> Csr:
  """`num_entries`: the valid entries of the buffers when known (it only
  picks kernel variants). `sorted_by_row` / `one_entry_per_row` set
  CSR_SORTED_BY_ROW / CSR_ONE_ENTRY_PER_ROW. `num_minibatches` > 0: the
  buffers are in the minibatching layout (row pointers of 64 blocks per
  segment); `positions_used` then bounds the positions holding entries (0:
  the whole buffer)."""
  rp_len = int(row_pointers.numel())
  if not 0 <= num_minibatches <= MAX_MINIBATCHES:
    raise ValueError("num_minibatches must be in [0, 64]")
  if num_minibatches:
    # max(NS, 8) row pointers per (SC, minibatch), packed from the start
    # (the buffer may be sized for 64 minibatches).
    per_block = max(num_partitions, 8)
    if rp_len < num_segments * num_minibatches * per_block:
      raise ValueError(
          f"row_pointers has {rp_len} entries; {num_minibatches} minibatches "
          f"of {num_segments} SparseCores need "
          f"{num_segments * num_minibatches * per_block}")
  else:
    if rp_len % num_segments:
      raise ValueError("row_pointers length must be divisible by "
                       "num_sc_per_device")
    per_block = rp_len // num_segments
  return Csr(ptr(row_pointers), ptr(embedding_ids), ptr(sample_ids),
             ptr(gains), int(embedding_ids.numel()), num_segments,
             num_partitions, per_block,
             (CSR_SORTED_BY_ROW if sorted_by_row else 0) |
             (CSR_ONE_ENTRY_PER_ROW if one_entry_per_row else 0),
             int(num_entries) if num_entries else 0, int(num_minibatches),
             int(positions_used) if num_minibatches else 0)


class LookupView:
  """Device buffers of a sample view (scemb_sample_view_t) plus the
  (device_batch_size, table_rows) pair it was built for."""

  def __init__(self, keys, entries, device_batch_size: int, table_rows: int,
               num_entries: int = 0, one_entry_per_key: bool = False):
    self.keys = keys          # int32 tensor holding the uint32 keys
    self.entries = entries    # int64 tensor holding the packed entries
    self.device_batch_size = int(device_batch_size)
    self.table_rows = int(table_rows)
    self.num_entries = int(num_entries)
    # No key twice (one-hot input rows): SCEMB_VIEW_ONE_ENTRY_PER_KEY.
    self.one_entry_per_key = bool(one_entry_per_key)

  def as_struct(self) -> SampleView:
    return SampleView(ptr(self.keys), ptr(self.entries),
                      int(self.keys.numel()), self.device_batch_size,
                      self.table_rows, self.num_entries,
                      VIEW_ONE_ENTRY_PER_KEY if self.one_entry_per_key else 0,
                      0)


def build_sample_view(csr: Csr, batch: int, table_rows: int,
                      device_status=None) -> LookupView:
  """Groups a CSR's entries by activation row (enqueued on the current
  stream; the CSR tensors must stay alive until it has run)."""
  t = require_gpu()
  lib = load_library()
  need = lib.scemb_build_sample_view_workspace_size(ctypes.byref(csr), batch,
                                                    table_rows)
  if need == 0:
    check(SCEMB_ERR_INVALID_ARGUMENT)
  n = int(csr.coo_size) // int(csr.num_segments) * int(csr.num_segments)
  keys = t.empty(n, dtype=t.int32, device=device())
  entries = t.empty(n, dtype=t.int64, device=device())
  ws = WORKSPACE.get(need)
  check(lib.scemb_build_sample_view(
      ctypes.byref(csr), batch, table_rows, ptr(keys), ptr(entries), ptr(ws),
      ws.numel(), ptr(device_status), stream_handle()))
  # A one-entry-per-row CSR is placed by activation row (a repeated row is
  # reported through STATUS_SHARED_ROW), so its view repeats no key.
  return LookupView(keys, entries, batch, table_rows, csr.num_entries,
                    one_entry_per_key=bool(csr.flags & CSR_ONE_ENTRY_PER_ROW))


def sparse_dense_matmul(csr: Csr | None, table, activations, batch: int,
                        view: LookupView | None = None,
                        device_status=None) -> None:
  lib = load_library()
  rows = int(table.shape[0])
  dim = 1 if table.dim() == 1 else int(table.shape[1])
  vs = view.as_struct() if view is not None else None
  csr_ref = ctypes.byref(csr) if csr is not None else None
  vs_ref = ctypes.byref(vs) if vs is not None else None
  need = lib.scemb_sparse_dense_matmul_workspace_size(csr_ref, vs_ref, batch,
                                                      rows, dim)
  if need == 0:
    check(SCEMB_ERR_INVALID_ARGUMENT)
  ws = WORKSPACE.get(need)
  check(lib.scemb_sparse_dense_matmul(
      csr_ref, vs_ref, ptr(table), rows, dim, ptr(activations), batch,
      ptr(ws), ws.numel(), ptr(device_status), stream_handle()))


def row_blocks(blocks) -> tuple:
  """ctypes array of RowBlock from (first_row, tensor, width) triples; each
  tensor is a CUDA float32 matrix whose rows are the block's rows."""
  arr = (RowBlock * max(len(blocks), 1))()
  for i, (first, t, width) in enumerate(blocks):
    arr[i] = RowBlock(int(first), int(t.shape[0]), ptr(t), int(t.stride(0)),
                      int(width), 0)
  return arr, len(blocks)


def sparse_dense_matmul_to_blocks(csr: Csr | None, table, blocks, batch: int,
                                  view: LookupView | None = None,
                                  device_status=None) -> None:
  """Forward lookup writing each activation row into its block (see
  scemb_row_block_t); `blocks` as for row_blocks."""
  lib = load_library()
  rows = int(table.shape[0])
  dim = 1 if table.dim() == 1 else int(table.shape[1])
  vs = view.as_struct() if view is not None else None
  csr_ref = ctypes.byref(csr) if csr is not None else None
  vs_ref = ctypes.byref(vs) if vs is not None else None
  need = lib.scemb_sparse_dense_matmul_workspace_size(csr_ref, vs_ref, batch,
                                                      rows, dim)
  if need == 0:
    check(SCEMB_ERR_INVALID_ARGUMENT)
  ws = WORKSPACE.get(need)
  arr, n = row_blocks(blocks)
  check(lib.scemb_sparse_dense_matmul_to_blocks(
      csr_ref, vs_ref, ptr(table), rows, dim, arr, n, batch, ptr(ws),
      ws.numel(), ptr(device_status), stream_handle()))


def activation_unstack(stacked, blocks) -> None:
  """Copies each block's stacked rows (first `width` columns) out of the
  [rows, dim] CUDA float32 matrix `stacked` into the block's tensor;
  `blocks` as for row_blocks."""
  arr, n = row_blocks(blocks)
  check(load_library().scemb_activation_unstack(
      ptr(stacked), int(stacked.shape[0]), int(stacked.shape[1]), arr, n,
      stream_handle()))


def gradient_stack(blocks, stacked) -> None:
  """Writes every row of the [rows, dim] CUDA float32 matrix `stacked`: a
  block's rows from its tensor's first `width` columns (zeros after them),
  rows in no block zero; `blocks` as for row_blocks."""
  arr, n = row_blocks(blocks)
  check(load_library().scemb_gradient_stack(
      arr, n, ptr(stacked), int(stacked.shape[0]), int(stacked.shape[1]),
      stream_handle()))


def _lr_args(learning_rate):
  t = torch()
  if isinstance(learning_rate, t.Tensor):
    lr = learning_rate.to(device=device(), dtype=t.float32).reshape(())
    return lr, ptr(lr), 0.0
  return None, None, float(np.float32(learning_rate))


def _clip_args(min_value, max_value):
  mask = (1 if min_value is not None else 0) | (2 if max_value is not None
                                                 else 0)
  return (mask, float(min_value) if min_value is not None else 0.0,
          float(max_value) if max_value is not None else 0.0)


def sparse_dense_matmul_grad(csr: Csr, activations_grad, table,
                             accumulator, learning_rate, batch: int,
                             min_value=None, max_value=None,
                             device_status=None, grad_blocks=None) -> None:
  """SGD when accumulator is None, Adagrad otherwise; updates in place.
  With `grad_blocks` ((first_row, tensor, width) triples, see row_blocks)
  the gradients are read from those per-feature blocks and
  `activations_grad` is ignored."""
  lib = load_library()
  rows = int(table.shape[0])
  dim = 1 if table.dim() == 1 else int(table.shape[1])
  need = lib.scemb_sparse_dense_matmul_grad_workspace_size(
      ctypes.byref(csr), batch, rows, dim)
  if need == 0:
    check(SCEMB_ERR_INVALID_ARGUMENT)
  ws = WORKSPACE.get(need)
  keep, lr_ptr, lr_val = _lr_args(learning_rate)
  mask, lo, hi = _clip_args(min_value, max_value)
  if grad_blocks is not None:
    arr, n = row_blocks(grad_blocks)
    if accumulator is None:
      rc = lib.scemb_sparse_dense_matmul_grad_with_sgd_from_blocks(
          ctypes.byref(csr), arr, n, batch, ptr(table), rows, dim, lr_ptr,
          lr_val, mask, lo, hi, ptr(ws), ws.numel(), ptr(device_status),
          stream_handle())
    else:
      rc = lib.scemb_sparse_dense_matmul_grad_with_adagrad_from_blocks(
          ctypes.byref(csr), arr, n, batch, ptr(table), ptr(accumulator),
          rows, dim, lr_ptr, lr_val, mask, lo, hi, ptr(ws), ws.numel(),
          ptr(device_status), stream_handle())
    del keep
    check(rc)
    return
  if accumulator is None:
    rc = lib.scemb_sparse_dense_matmul_grad_with_sgd(
        ctypes.byref(csr), ptr(activations_grad), batch, ptr(table), rows, dim,
        lr_ptr, lr_val, mask, lo, hi, ptr(ws), ws.numel(), ptr(device_status),
        stream_handle())
  else:
    rc = lib.scemb_sparse_dense_matmul_grad_with_adagrad(
        ctypes.byref(csr), ptr(activations_grad), batch, ptr(table),
        ptr(accumulator), rows, dim, lr_ptr, lr_val, mask, lo, hi, ptr(ws),
        ws.numel(), ptr(device_status), stream_handle())
  del keep
  check(rc)


def _hyper_args(values):
  """Device scalars stay on the device (passed by pointer, read by the
  kernels); anything else becomes a float32 value."""
  t = torch()
  keep, ptrs, vals = [], [], []
  for v in values:
    if isinstance(v, t.Tensor):
      d = v.to(device=device(), dtype=t.float32).reshape(())
      keep.append(d)
      ptrs.append(ptr(d))
      vals.append(0.0)
    else:
      ptrs.append(None)
      vals.append(float(np.float32(np.asarray(v, np.float32))))
  return keep, ptrs, vals


def sparse_dense_matmul_grad_with_optimizer(
    csr: Csr, activations_grad, table, kind: int, slots, hyperparameters,
    batch: int, min_value=None, max_value=None, flags: int = 0,
    device_status=None, grad_blocks=None, program=None) -> None:
  """Backward + the optimizer `kind` (OPTIMIZER_*), updating `table` and the
  slot tensors in place. `hyperparameters` in the order of the reference
  primitive's operands (floats, numpy scalars or 0-d tensors).
  `grad_blocks`: as for sparse_dense_matmul_grad. `program`: the
  UpdateProgram struct of OPTIMIZER_CUSTOM."""
  lib = load_library()
  if len(hyperparameters) > MAX_HYPERPARAMETERS or len(slots) > 2:
    check(SCEMB_ERR_INVALID_ARGUMENT)
  rows = int(table.shape[0])
  dim = 1 if table.dim() == 1 else int(table.shape[1])
  need = lib.scemb_sparse_dense_matmul_grad_workspace_size(
      ctypes.byref(csr), batch, rows, dim)
  if need == 0:
    check(SCEMB_ERR_INVALID_ARGUMENT)
  ws = WORKSPACE.get(need)
  keep, hp_ptrs, hp_vals = _hyper_args(hyperparameters)
  opt = Optimizer()
  opt.kind = kind
  opt.flags = flags
  for i, s in enumerate(slots):
    opt.slots[i] = ptr(s)
  for i, (p, v) in enumerate(zip(hp_ptrs, hp_vals)):
    opt.hyperparameter_ptrs[i] = p
    opt.hyperparameters[i] = v
  opt.clip_mask, opt.min_value, opt.max_value = _clip_args(min_value,
                                                           max_value)
  if program is not None:
    opt.program = ctypes.pointer(program)
  if grad_blocks is not None:
    arr, n = row_blocks(grad_blocks)
    rc = lib.scemb_sparse_dense_matmul_grad_with_optimizer_from_blocks(
        ctypes.byref(csr), arr, n, batch, ptr(table), rows, dim,
        ctypes.byref(opt), ptr(ws), ws.numel(), ptr(device_status),
        stream_handle())
  else:
    rc = lib.scemb_sparse_dense_matmul_grad_with_optimizer(
        ctypes.byref(csr), ptr(activations_grad), batch, ptr(table), rows,
        dim, ctypes.byref(opt), ptr(ws), ws.numel(), ptr(device_status),
        stream_handle())
  del keep
  check(rc)
