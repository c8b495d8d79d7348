"""FDO client storing stats as .csv files (reference:
lib/fdo/csv_file_fdo_client.py:33-216): a ``key,values`` header, then one
line per key and recorded batch with the values separated by spaces."""

from __future__ import annotations

import csv
import os

import numpy as np

from jax_tpu_embedding.sparsecore.lib.fdo import fdo_client


class CSVFileFDOClient(fdo_client.FileStatsStore):
  """As NPZFileFDOClient, in CSV. With ``retain_history=False`` each
  ``record`` keeps only the element-wise maximum over the batches recorded so
  far instead of one row per batch."""

  extension = "csv"

  def __init__(self, base_dir: str | os.PathLike, retain_history: bool = True):
    super().__init__(base_dir)
    self._retain_history = retain_history

  def record(self, data):
    super().record(data)
    if self._retain_history:
      return
    for name, per_table in self._params.items():
      self._params[name] = {
          table: (np.max(v, axis=0) if v.ndim > 1 else v)
          for table, v in per_table.items()}

  def _write(self, file_name, stats):
    with open(file_name, "w", newline="") as f:
      w = csv.writer(f)
      w.writerow(["key", "values"])
      for key, array in stats.items():
        array = np.asarray(array, np.int64)
        rows = array.reshape(1, -1) if array.ndim <= 1 else array
        for row in rows:
          w.writerow([key, " ".join(str(int(x)) for x in row)])

  def _read(self, file_name):
    lines: dict[str, list[np.ndarray]] = {}
    with open(file_name, newline="") as f:
      reader = csv.reader(f)
      next(reader)  # header
      for row in reader:
        if not row:
          continue
        key, text = row
        lines.setdefault(key, []).append(
            np.array([int(x) for x in text.split()], dtype=np.int64))
    return {key: (np.vstack(v) if len(v) > 1 else v[0])
            for key, v in lines.items()}
