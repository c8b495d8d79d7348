"""Shared pytest setup: import paths and the `gpu` marker."""

import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_PKG_ROOT = os.path.join(_ROOT, "jax-tpu-embedding_amd")
for p in (_ROOT, _PKG_ROOT):
  if p not in sys.path:
    sys.path.insert(0, p)


def pytest_configure(config):
  config.addinivalue_line(
      "markers", "gpu: needs an MI355X (runs through libscemb.so on cuda:0)")
