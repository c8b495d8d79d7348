"""Constants shared with the reference (lib/core/constants.py:17)."""

# Value written to the embedding and sample ids of alignment padding slots in
# the CSR buffers (input_preprocessing_util.cc:126-131).
PADDING_VALUE = 2**31 - 1
