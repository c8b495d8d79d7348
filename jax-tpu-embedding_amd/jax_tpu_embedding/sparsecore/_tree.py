"""Minimal pytree helpers for nested feature / table / array collections.

Follows jax.tree's conventions for the containers the embedding API uses:
lists, tuples and NamedTuples flatten in order, dicts flatten by sorted key,
``None`` is an empty subtree, anything else is a leaf.
"""

from __future__ import annotations

from typing import Any, Callable


def _is_namedtuple(x) -> bool:
  return isinstance(x, tuple) and hasattr(x, "_fields")


def tree_flatten(tree) -> tuple[list, Any]:
  leaves: list = []

  def rec(x):
    if x is None:
      return ("none",)
    if isinstance(x, dict):
      keys = sorted(x.keys())
      return ("dict", tuple(keys), tuple(rec(x[k]) for k in keys))
    if _is_namedtuple(x):
      return ("namedtuple", type(x), tuple(rec(v) for v in x))
    if isinstance(x, (list, tuple)):
      return (type(x).__name__, tuple(rec(v) for v in x))
    leaves.append(x)
    return ("leaf",)

  treedef = rec(tree)
  return leaves, treedef


def tree_unflatten(treedef, leaves) -> Any:
  it = iter(leaves)

  def rec(d):
    kind = d[0]
    if kind == "none":
      return None
    if kind == "leaf":
      return next(it)
    if kind == "dict":
      return {k: rec(c) for k, c in zip(d[1], d[2])}
    if kind == "namedtuple":
      return d[1](*[rec(c) for c in d[2]])
    children = [rec(c) for c in d[1]]
    return children if kind == "list" else tuple(children)

  return rec(treedef)


def _flat_leaves(tree) -> bool:
  """Whether tree is a plain list or tuple of leaves (the common case, which
  needs no walk)."""
  if type(tree) not in (list, tuple):
    return False
  for v in tree:
    if v is None or isinstance(v, (dict, list, tuple)):
      return False
  return True


def tree_leaves(tree) -> list:
  """The leaves of tree_flatten, without building the structure."""
  if _flat_leaves(tree):
    return list(tree)
  leaves: list = []

  def rec(x):
    if x is None:
      return
    if isinstance(x, dict):
      for k in sorted(x.keys()):
        rec(x[k])
    elif isinstance(x, (list, tuple)):  # NamedTuples included, in order
      for v in x:
        rec(v)
    else:
      leaves.append(x)

  rec(tree)
  return leaves


def tree_structure(tree):
  return tree_flatten(tree)[1]


def tree_map(fn: Callable, tree, *rest) -> Any:
  leaves, treedef = tree_flatten(tree)
  others = [tree_flatten(r)[0] for r in rest]
  return tree_unflatten(treedef,
                        [fn(*xs) for xs in zip(leaves, *others)])


def leaf_paths(tree) -> list:
  """Paths (tuples of keys / indices) of the leaves, in flattening order."""
  if _flat_leaves(tree):
    return [(i,) for i in range(len(tree))]
  out = []

  def rec(x, path):
    if x is None:
      return
    if isinstance(x, dict):
      for k in sorted(x.keys()):
        rec(x[k], path + (k,))
    elif isinstance(x, (list, tuple)):
      for i, v in enumerate(x):
        rec(v, path + (i,))
    else:
      out.append(path)

  rec(tree, ())
  return out
