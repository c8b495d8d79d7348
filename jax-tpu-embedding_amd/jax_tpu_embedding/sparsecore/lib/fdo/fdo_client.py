"""FDO client interface and the file-store logic shared by the NPZ and CSV
clients (reference: lib/fdo/fdo_client.py:23-83, file_fdo_client.py,
csv_file_fdo_client.py).

Storage layout, kept identical to the reference's so that stats files move
between the two implementations: every process writes
``fdo_stats_<process index>_<time in ns>.<ext>`` into a base directory, with
one entry per (stacked table, stat) named ``<table><suffix>`` (the suffixes
are the metadata of SparseDenseMatmulInputStats' fields). ``load`` reads the
newest file of every process and takes the element-wise maximum across
processes.
"""

from __future__ import annotations

import abc
import dataclasses
import itertools
import logging
import os
import pathlib
import re
import time

import numpy as np

from jax_tpu_embedding.sparsecore.lib.nn import embedding

FILE_NAME = "fdo_stats"
_STAT_FIELDS = dataclasses.fields(embedding.SparseDenseMatmulInputStats)


class FDOClient(abc.ABC):
  """Per-process client of an FDO store.

  1. ``record`` the stats of one or more preprocessed batches;
  2. ``publish`` them to the store;
  3. ``load`` the stats aggregated over every process that published.
  """

  @abc.abstractmethod
  def record(self, data: embedding.SparseDenseMatmulInputStats) -> None:
    raise NotImplementedError

  @abc.abstractmethod
  def publish(self) -> None:
    raise NotImplementedError

  @abc.abstractmethod
  def load(self) -> embedding.SparseDenseMatmulInputStats:
    raise NotImplementedError


def process_index() -> int:
  """This process's rank among the trainer processes (jax.process_index in
  the reference): the torch.distributed rank when a process group is up,
  else 0."""
  try:
    import torch.distributed as dist  # pylint: disable=g-import-not-at-top
    if dist.is_available() and dist.is_initialized():
      return int(dist.get_rank())
  except ImportError:
    pass
  return 0


class FileStatsStore(FDOClient):
  """Record / publish / load over files of one format; subclasses write and
  read a {key: int64 array} mapping (`_write`, `_read`)."""

  extension = ""

  def __init__(self, base_dir: str | os.PathLike):
    self._base_dir = pathlib.Path(base_dir)
    # stat field -> table -> int64 array (one row per recorded batch).
    self._params: dict[str, dict[str, np.ndarray]] = {
        f.name: {} for f in _STAT_FIELDS}

  # -- recording ------------------------------------------------------------

  def record(self, data: embedding.SparseDenseMatmulInputStats) -> None:
    """Appends the stats of one batch (a new row per table and stat)."""
    for name, per_table in dataclasses.asdict(data).items():
      if name not in self._params:
        logging.warning("Unsupported FDO stats: %s", name)
        continue
      for table, value in per_table.items():
        value = np.asarray(value, dtype=np.int64)
        held = self._params[name].get(table)
        self._params[name][table] = (value if held is None else
                                     np.vstack((held, value)))

  def _keyed(self) -> dict[str, np.ndarray]:
    out = {}
    for f in _STAT_FIELDS:
      for table, value in self._params[f.name].items():
        out[f"{table}{f.metadata['suffix']}"] = value
    return out

  # -- files ----------------------------------------------------------------

  def _new_file_name(self) -> str:
    return os.fspath(self._base_dir / (
        f"{FILE_NAME}_{process_index()}_{time.time_ns()}.{self.extension}"))

  def _get_latest_files_by_process(self, files: list[str]) -> list[str]:
    """The newest file of each process, processes in descending order of
    their index (compared as text, like the reference)."""
    pattern = re.compile(rf"{FILE_NAME}_(\d+)_(\d+)\.{self.extension}$")
    found = []
    for f in files:
      m = pattern.search(os.path.basename(f))
      if m:
        found.append((m.group(1), int(m.group(2)), f))
    found.sort(reverse=True)
    return [next(group)[2]
            for _, group in itertools.groupby(found, key=lambda x: x[0])]

  def publish(self) -> None:
    name = self._new_file_name()
    logging.info("Write stats to %s", name)
    self._write(name, self._keyed())

  def load(self) -> embedding.SparseDenseMatmulInputStats:
    pattern = os.fspath(self._base_dir / f"{FILE_NAME}*.{self.extension}")
    files = self._get_latest_files_by_process(
        [os.fspath(p) for p in self._base_dir.glob(
            f"{FILE_NAME}*.{self.extension}")])
    if not files:
      raise FileNotFoundError(f"No stats files found in {pattern}")
    merged: dict[str, np.ndarray] = {}
    for name in files:
      logging.info("Reading stats from %s", name)
      for key, value in self._read(name).items():
        held = merged.get(key)
        merged[key] = (value if held is None else
                       np.max(np.vstack((held, value)), axis=0))
    result: dict[str, dict[str, np.ndarray]] = {
        f.name: {} for f in _STAT_FIELDS}
    for key, value in merged.items():
      for f in _STAT_FIELDS:
        suffix = f.metadata["suffix"]
        if key.endswith(suffix):
          result[f.name][key[:-len(suffix)]] = value
          break
      else:
        raise ValueError(
            f"Unexpected key: {key}, expected to end with "
            f"{[f.metadata['suffix'] for f in _STAT_FIELDS]}")
    self._params = result
    return embedding.SparseDenseMatmulInputStats(**result)

  @abc.abstractmethod
  def _write(self, file_name: str, stats: dict[str, np.ndarray]) -> None:
    raise NotImplementedError

  @abc.abstractmethod
  def _read(self, file_name: str) -> dict[str, np.ndarray]:
    raise NotImplementedError

