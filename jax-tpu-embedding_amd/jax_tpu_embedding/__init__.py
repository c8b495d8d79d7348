"""MI355X-native drop-in for jax_tpu_embedding's SparseCore embedding path.

The module layout mirrors the reference package
(``jax_tpu_embedding.sparsecore.lib.nn.embedding`` and friends) so existing
imports keep working; arrays are torch tensors on the GPU and the compute runs
in ``libscemb.so`` (hand-written gfx950 HIP kernels).
"""
