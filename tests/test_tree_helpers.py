"""The pytree helpers: tree_leaves and leaf_paths (which take a fast path
for flat lists and tuples of leaves) agree with tree_flatten's leaves and
with a plain recursive walk, for the containers the embedding API accepts:
lists, tuples, NamedTuples, dicts (sorted keys) and None (empty)."""

import collections

import numpy as np

from jax_tpu_embedding.sparsecore import _tree

_NT = collections.namedtuple("_NT", "a b")

TREES = [
    [1, 2, 3], (1, 2), [], (), None, 5, np.zeros(3),
    {"b": [1, None, 2], "a": (3, _NT(4, [5, 6]))},
    [np.zeros(2), np.ones(3)], [[1], [2, 3]], _NT(1, 2), [None, 1],
    {"x": 1}, [{"a": 1}], (1, (2,)), [_NT(1, 2), 3],
]


def _walk_paths(tree):
  out = []

  def rec(x, path):
    if x is None:
      return
    if isinstance(x, dict):
      for k in sorted(x):
        rec(x[k], path + (k,))
    elif isinstance(x, (list, tuple)):
      for i, v in enumerate(x):
        rec(v, path + (i,))
    else:
      out.append(path)

  rec(tree, ())
  return out


def test_leaves_and_paths_match_the_full_flatten():
  for tree in TREES:
    leaves = _tree.tree_leaves(tree)
    want = _tree.tree_flatten(tree)[0]
    assert len(leaves) == len(want)
    assert all(a is b for a, b in zip(leaves, want)), tree
    assert _tree.leaf_paths(tree) == _walk_paths(tree), tree


def test_round_trip():
  for tree in TREES:
    leaves, treedef = _tree.tree_flatten(tree)
    back = _tree.tree_unflatten(treedef, leaves)
    assert _tree.tree_flatten(back)[1] == treedef
