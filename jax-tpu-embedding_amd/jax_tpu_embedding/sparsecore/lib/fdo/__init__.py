"""Feedback-directed optimisation (FDO) of the preprocessing limits: stats
observed by preprocess_sparse_dense_matmul_input are recorded per process,
published to shared storage and loaded back aggregated over processes, to
feed embedding.update_preprocessing_parameters (reference: lib/fdo/)."""
