"""Device utilities (reference: jax_tpu_embedding/sparsecore/utils/utils.py).

``NUM_SC_PER_DEVICE_MAP`` keeps the TPU entries of the reference (:30-36) and
adds the MI355X: one GPU runs the path as a single SparseCore-equivalent CSR
segment, so its count is 1. ``shard_emb_table`` / ``unshard_emb_table`` are the
MOD layout of :90-136 (a row permutation), written with einops for numpy
arrays and torch tensors.
"""

from __future__ import annotations

import typing

import einops

NUM_SC_PER_DEVICE_MAP = {
    "TPU v5": 4,
    "TPU v5p": 4,
    "TPU v6e": 2,
    "TPU v6 lite": 2,
    "TPU7x": 2,
    "AMD Instinct MI355X": 1,
}


class DeviceLike(typing.Protocol):

  @property
  def device_kind(self) -> str:
    ...


def _device_kind(device) -> str:
  if device is not None and hasattr(device, "device_kind"):
    return device.device_kind
  import torch  # pylint: disable=g-import-not-at-top

  index = None
  if device is not None and hasattr(device, "index"):
    index = device.index
  if not torch.cuda.is_available():
    raise ValueError("Cannot determine device kind: no GPU is visible.")
  i = index if index is not None else 0
  name = torch.cuda.get_device_name(i)
  # Some ROCm installs report a generic marketing name ("AMD Radeon
  # Graphics"); the architecture name identifies the MI355X (gfx950).
  arch = getattr(torch.cuda.get_device_properties(i), "gcnArchName", "") or ""
  if "MI355" not in name and arch.split(":")[0] == "gfx950":
    return "AMD Instinct MI355X"
  return name


def num_sparsecores_per_device(device: DeviceLike | None = None) -> int:
  """SparseCore count of `device` (default: the current GPU).

  Raises:
    ValueError: if the device kind is unknown.
  """
  kind = _device_kind(device)
  if kind in NUM_SC_PER_DEVICE_MAP:
    return NUM_SC_PER_DEVICE_MAP[kind]
  if "MI355" in kind:
    return NUM_SC_PER_DEVICE_MAP["AMD Instinct MI355X"]
  raise ValueError(
      f"Unknown sparsecore count for device kind: {kind}. Known device kinds: "
      f"{NUM_SC_PER_DEVICE_MAP.keys()}")


def shard_emb_table(table, *, num_devices: int, num_sc_per_device: int,
                    sharding_strategy: str = "MOD"):
  """[vocab, dim] -> [num_devices, num_sc_per_device * vocab_per_sc, dim]."""
  if sharding_strategy != "MOD":
    raise ValueError("Currently only MOD sharding strategy is supported")
  return einops.rearrange(table, "(v c s) ... -> c (s v) ...", c=num_devices,
                          s=num_sc_per_device)


def unshard_emb_table(sharded_table, num_sc_per_device: int,
                      sharding_strategy: str = "MOD"):
  """Inverse of shard_emb_table."""
  if sharding_strategy != "MOD":
    raise ValueError("Currently only MOD sharding strategy is supported")
  return einops.rearrange(sharded_table, "c (s v) ... -> (v c s) ...",
                          s=num_sc_per_device)
