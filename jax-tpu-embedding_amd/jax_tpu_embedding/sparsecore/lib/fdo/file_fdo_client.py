"""FDO client storing stats as .npz files (reference:
lib/fdo/file_fdo_client.py:33-213): one array per ``<table><suffix>`` key,
one row per recorded batch."""

from __future__ import annotations

import numpy as np

from jax_tpu_embedding.sparsecore.lib.fdo import fdo_client


class NPZFileFDOClient(fdo_client.FileStatsStore):
  """Usage:

    client = NPZFileFDOClient(base_dir)
    _, stats = embedding.preprocess_sparse_dense_matmul_input(...)
    client.record(stats)
    client.publish()
    stats = client.load()   # max over the newest file of every process
  """

  extension = "npz"

  def _write(self, file_name, stats):
    np.savez(file_name, **stats)

  def _read(self, file_name):
    with np.load(file_name, allow_pickle=False) as loaded:
      return {key: loaded[key] for key in loaded.files}
