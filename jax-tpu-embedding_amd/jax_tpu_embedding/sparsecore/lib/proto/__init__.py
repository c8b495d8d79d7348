"""Embedding spec messages (reference: lib/proto/embedding_spec.proto)."""
