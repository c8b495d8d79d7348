/* scemb.h - C ABI of libscemb, the MI355X (gfx950) SparseCore embedding path.
 *
 * Plain pointers and sizes only. Device pointers are HIP device memory; the
 * `stream` arguments are hipStream_t values passed as void*. Every entry point
 * only enqueues work on `stream` (no host synchronisation, no allocation
 * beyond the caller's workspace) unless its comment says otherwise, and
 * returns SCEMB_OK or an error code with a message in scemb_last_error().
 * Nothing in the library aborts the process.
 *
 * Reference interfaces replaced (paths relative to
 * jax_tpu_embedding/sparsecore/ in jax-ml/jax-tpu-embedding):
 *   scemb_sparse_dense_matmul              custom call "SparseDenseMatmulOp",
 *       lowered at lib/core/primitives/sparse_dense_matmul_csr.py:171-201
 *   scemb_build_sample_view                no counterpart (the SparseCore
 *       groups by sample in hardware); optional input of the forward
 *   scemb_*_to_blocks / *_from_blocks       the same ops with the activation
 *       unstacking (lib/nn/embedding.py:903-1044) and gradient stacking
 *       (:1200-1294) fused in: per-feature row blocks instead of one stacked
 *       matrix
 *   scemb_sparse_dense_matmul_grad_with_sgd  custom call
 *       "SparseDenseMatmulGradOpWithOptimizerUpdate" with the SGD update
 *       computation, lib/core/primitives/sparse_dense_matmul_grad_with_sgd.py:
 *       194-227 (update fn :145-192)
 *   scemb_sparse_dense_matmul_grad_with_adagrad  the same custom call with
 *       the Adagrad update, lib/core/primitives/
 *       sparse_dense_matmul_grad_with_adagrad.py:235-275 (update fn :167-233)
 *   scemb_sparse_dense_matmul_grad_with_optimizer  the same custom call for
 *       every built-in optimizer (Adam, AdagradMomentum, FTRL, LaProp, F2A,
 *       and SGD / Adagrad), lib/core/primitives/
 *       sparse_dense_matmul_grad_with_{adam,adagrad_momentum,ftrl,laprop,
 *       f2a}.py (each file's lowering and update function)
 *   scemb_preprocess_stacked_table         PreprocessSparseDenseMatmulInput
 *       for one stacked table, lib/core/input_preprocessing.h:62-68 /
 *       input_preprocessing.cc:800-959, as bound by
 *       lib/core/pybind_input_preprocessing.cc:124-188
 *   scemb_compute_*                         size helpers of
 *       lib/core/pybind_input_preprocessing.cc:203-262 (bound at :311-320)
 */
#ifndef SCEMB_H_
#define SCEMB_H_

#ifndef __HIPCC_RTC__ /* kernels compiled at run time get these types built in */
#include <stddef.h>
#include <stdint.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define SCEMB_OK 0
#define SCEMB_ERR_INVALID_ARGUMENT 1 /* Python: ValueError */
#define SCEMB_ERR_NOT_IMPLEMENTED 2
#define SCEMB_ERR_WORKSPACE 3        /* workspace missing or too small */
#define SCEMB_ERR_DEVICE 4           /* HIP runtime error */
#define SCEMB_ERR_LIMIT_EXCEEDED 5   /* ids over the partition limits with
                                        dropping disabled (the reference
                                        LOG(FATAL)s); Python: RuntimeError */

/* Bits OR-ed into the optional device status word by the kernels. */
#define SCEMB_STATUS_BAD_ENTRY 1u    /* CSR entry with an embedding id or
                                        sample id out of range: skipped */
#define SCEMB_STATUS_BAD_ID 2u       /* preprocessing input id outside
                                        [0, col_id_bound): skipped */
#define SCEMB_STATUS_UNSORTED 4u     /* a stream declared sorted (CSR flag
                                        or sample view) is not: results are
                                        not valid */
#define SCEMB_STATUS_SHARED_ROW 8u   /* a CSR declared with at most one
                                        entry per activation row has two:
                                        results are not valid */

/* Message of the last failing call on this thread ("" if none). */
const char* scemb_last_error(void);

/* Library version, (major << 16) | minor. */
int scemb_version(void);

/* One device's CSR-wrapped COO buffers for one stacked table
 * (SparseDenseMatmulInput; layout documented at
 * lib/core/input_preprocessing_util.cc:167-208). For local SparseCore s and
 * partition p, entries j in [roundup8(rp[s*R + p - 1]) (0 for p = 0),
 * rp[s*R + p]) of segment s (positions s*coo_size/num_segments + j) hold
 * (embedding id, sample id, gain).
 *
 * With num_minibatches > 0 the buffers are in the minibatching layout
 * (enable_minibatching; input_preprocessing_util.cc:135-143, :331-473, the
 * operands of "SparseDenseMatmulWithMinibatchingOp",
 * primitives/sparse_dense_matmul_csr.py:171-192): segment s holds
 * num_minibatches blocks of R row pointers (block b = s * num_minibatches +
 * m at rp[b*R]), row pointers are positions in the whole buffer, and each
 * partition's entries start at the aligned end of the partition before it
 * in buffer order (the first at 0). */
typedef struct scemb_csr {
  const int32_t* row_pointers;  /* [num_segments * row_pointers_per_segment]
                                   (times num_minibatches when > 0) */
  const int32_t* embedding_ids; /* [coo_size] */
  const int32_t* sample_ids;    /* [coo_size] */
  const float* gains;           /* [coo_size] */
  int64_t coo_size;
  int32_t num_segments;             /* num_sc_per_device */
  int32_t num_partitions;           /* num_sc_per_device * global devices */
  int32_t row_pointers_per_segment; /* max(num_partitions, 8) */
  uint32_t flags;                   /* SCEMB_CSR_* bits */
  int64_t num_entries; /* valid entries if known (> 0), else 0: only picks
                          kernel variants (about one entry per activation
                          row or more); the buffer size stands in when 0 */
  int32_t num_minibatches; /* 0: one block per segment (no minibatching);
                              1..64: the minibatching layout */
  int32_t positions_used;  /* minibatching layout: every entry lies below
                              this buffer position (0: anywhere below
                              coo_size). The buffer is sized for 64
                              minibatches; a bound from the preprocessing
                              (entries + 7 per (SC, minibatch, partition),
                              rounded up to 8) spares the lookup the rest. */
} scemb_csr_t;

/* The entries of each segment are ascending by (partition, embedding id), as
 * the preprocessing writes them (input_preprocessing_util.cc:167-208 sorts by
 * the rotated column id). With one segment the backward pass then reads the
 * CSR in place instead of sorting it; order violations are reported through
 * SCEMB_STATUS_UNSORTED. In the minibatching layout the flag declares that
 * every table row's entries are contiguous (one local SparseCore: a column
 * falls in one bucket, so in one minibatch, where it is sorted), which is not
 * checked. */
#define SCEMB_CSR_SORTED_BY_ROW 1u

/* At most one valid entry per activation row (every input row of the stack
 * holds at most one id: one-hot features). Building the sample view is then
 * a placement by activation row instead of a sort; a second entry for a row
 * is reported through SCEMB_STATUS_SHARED_ROW. */
#define SCEMB_CSR_ONE_ENTRY_PER_ROW 2u

/* The CSR entries of one device grouped by activation row (no counterpart
 * in the reference, where the SparseCore scatters into activations in
 * hardware): entry i adds gain_i * table[row_i] to activations[keys[i]].
 * keys are ascending, entries of one key keep CSR order, keys >=
 * device_batch_size mark unused slots (at the end). entries[i] packs
 * row_i | (IEEE bits of gain_i) << 32. Built by scemb_build_sample_view for
 * one (device_batch_size, table_rows) pair; the forward pass checks both. */
typedef struct scemb_sample_view {
  const uint32_t* keys;     /* [size] */
  const uint64_t* entries;  /* [size] */
  int64_t size;
  int64_t device_batch_size;
  int64_t table_rows;
  int64_t num_entries;      /* as scemb_csr_t.num_entries */
  uint32_t flags;           /* SCEMB_VIEW_* bits */
  int32_t reserved;
} scemb_sample_view_t;

/* No key appears twice (the view of a CSR with SCEMB_CSR_ONE_ENTRY_PER_ROW):
 * no activation row's sum crosses a work-group, so the forward pass skips its
 * cross-block combining launch. A repeated key is reported through
 * SCEMB_STATUS_SHARED_ROW (results are then not valid). */
#define SCEMB_VIEW_ONE_ENTRY_PER_KEY 1u

/* One feature's rows of a stacked activation (or activation-gradient)
 * matrix of device_batch_size x dim: stacked rows [first_row, first_row +
 * num_rows) are rows 0.. of `data`, row_stride floats apart, holding the
 * first `width` columns (the feature's own dim; the remaining dim - width
 * are stacking padding: the forward does not write them, the backward reads
 * them as zero). Blocks are ascending in first_row and disjoint; rows in no
 * block are not written (forward) or contribute nothing (backward). */
typedef struct scemb_row_block {
  int64_t first_row;
  int64_t num_rows;
  float* data;
  int64_t row_stride;
  int32_t width;
  int32_t reserved;
} scemb_row_block_t;
#define SCEMB_MAX_ROW_BLOCKS 32

/* ---- Forward: SparseDenseMatmulOp --------------------------------------
 * activations[b, :] = sum over entries with s*bps + sample_id == b of
 *   gain * table[p * (table_rows / num_partitions) + embedding_id, :],
 * bps = device_batch_size / num_segments; rows without entries are zero.
 * `table` is [table_rows, dim] row-major (dim 1 for a 1-D table). Entries
 * whose ids fall outside the table or batch are skipped and flagged in
 * *device_status (optional, may be NULL). When `view` is not NULL the CSR
 * is not read (csr may be NULL) and the view's entries are used instead;
 * otherwise the call builds the same grouping itself. Each row is summed in
 * a fixed order: pieces of consecutive entries in CSR order, added in a
 * fixed tree, so repeated calls give identical results. */
size_t scemb_sparse_dense_matmul_workspace_size(const scemb_csr_t* csr,
                                                const scemb_sample_view_t* view,
                                                int64_t device_batch_size,
                                                int64_t table_rows,
                                                int32_t dim);
int scemb_sparse_dense_matmul(const scemb_csr_t* csr,
                              const scemb_sample_view_t* view,
                              const float* table, int64_t table_rows,
                              int32_t dim, float* activations,
                              int64_t device_batch_size, void* workspace,
                              size_t workspace_bytes, uint32_t* device_status,
                              void* stream);
/* No counterpart in the reference. The same lookup for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): no workspace argument and no allocation; its
 * scratch is a library-owned device array of SCEMB_NO_ALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends. A lookup whose workspace
 * (scemb_sparse_dense_matmul_workspace_size) exceeds that returns
 * SCEMB_ERR_INVALID_ARGUMENT. Every call on a GPU uses that GPU's one
 * array: calls that overlap on one GPU (different streams or host threads)
 * race and must be serialised by the caller. Results equal those of
 * scemb_sparse_dense_matmul bit for bit. */
#define SCEMB_NO_ALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int scemb_sparse_dense_matmul_no_alloc(const scemb_csr_t* csr,
                                       const scemb_sample_view_t* view,
                                       const float* table, int64_t table_rows,
                                       int32_t dim, float* activations,
                                       int64_t device_batch_size,
                                       uint32_t* device_status, void* stream);
/* The same, writing each activation row into its feature's block (the
 * unstacked per-feature outputs); workspace as for the call above. */
int scemb_sparse_dense_matmul_to_blocks(
    const scemb_csr_t* csr, const scemb_sample_view_t* view,
    const float* table, int64_t table_rows, int32_t dim,
    const scemb_row_block_t* outputs, int32_t num_outputs,
    int64_t device_batch_size, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream);

/* ---- SparseActivationsUnstackInterleaved --------------------------------
 * Replaces the custom call of tpu_sparse_dense_matmul_activation_unstack_
 * primitive (lib/core/primitives/sparse_dense_matmul_activation_unstack.py:
 * 64-96 of the reference). For each block, stacked rows [first_row,
 * first_row + num_rows), columns [0, width), of `stacked` ([rows, dim]
 * row-major) are copied to the block's rows. With several SparseCores a
 * feature takes one block per SparseCore (its slice of each segment); blocks
 * may come in any order and any number. Only enqueues on `stream`. */
int scemb_activation_unstack(const float* stacked, int64_t rows, int32_t dim,
                             const scemb_row_block_t* blocks,
                             int32_t num_blocks, void* stream);

/* ---- SparseGradientsStackInterleaved ------------------------------------
 * Replaces the custom call of tpu_sparse_dense_matmul_gradient_stack_
 * primitive (lib/core/primitives/sparse_dense_matmul_gradient_stack.py:
 * 46-86 of the reference). Writes every row of `stacked` ([rows, dim]
 * row-major): a row of a block gets the block's first `width` columns and
 * zeros after them; a row in no block is zero. Blocks must not overlap.
 * Only enqueues on `stream`. */
int scemb_gradient_stack(const scemb_row_block_t* blocks, int32_t num_blocks,
                         float* stacked, int64_t rows, int32_t dim,
                         void* stream);

/* Builds the sample view of a CSR into keys[coo_size] / entries[coo_size]
 * (device memory owned by the caller). Invalid entries are flagged as in the
 * forward pass and left out of the view. */
size_t scemb_build_sample_view_workspace_size(const scemb_csr_t* csr,
                                              int64_t device_batch_size,
                                              int64_t table_rows);
int scemb_build_sample_view(const scemb_csr_t* csr, int64_t device_batch_size,
                            int64_t table_rows, uint32_t* keys,
                            uint64_t* entries, void* workspace,
                            size_t workspace_bytes, uint32_t* device_status,
                            void* stream);

/* ---- Backward + optimizer: SparseDenseMatmulGradOpWithOptimizerUpdate ----
 * For every touched table row r:
 *   g_r = sum over its entries of gain * activations_grad[s*bps + sample_id]
 * then, once per touched row (untouched rows are not modified),
 *   SGD:     T[r] = T[r] - g_r * lr
 *   Adagrad: A[r] = A[r] + g_r * g_r;  T[r] = T[r] - (lr * g_r) / sqrt(A[r])
 * followed by T[r] = clamp(T[r], min, max) for the bounds that are given
 * (clip_mask bit 0: min_value, bit 1: max_value). Tables are updated in
 * place. The learning rate is read from `learning_rate` (device scalar) when
 * not NULL, else `learning_rate_value` is used. No float atomics: every
 * row's gradient is summed in a fixed order (pieces of consecutive entries,
 * added in a fixed tree) and the row is updated once. With
 * SCEMB_CSR_SORTED_BY_ROW and one segment the CSR is read in place; else the
 * call sorts a copy of the entries by table row. A CSR read in place
 * without minibatching, with several entries per activation row, may have
 * its long runs (entries ascending by sample, checked) reduced per sample
 * tile instead. The tile sums use fused multiply-adds: the same fixed-order
 * guarantee, different rounding. The environment variables
 * SCEMB_HOT_RUNS (0 off, 1 whenever eligible, unset: activation gradients
 * over 64 MB and tiles of 128 samples or more) and SCEMB_HOT_MAX_RUNS decide
 * it. The workspace size then includes its buffers, so they must not change
 * between sizing and the call. */
size_t scemb_sparse_dense_matmul_grad_workspace_size(const scemb_csr_t* csr,
                                                     int64_t device_batch_size,
                                                     int64_t table_rows,
                                                     int32_t dim);
int scemb_sparse_dense_matmul_grad_with_sgd(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, int64_t table_rows, int32_t dim,
    const float* learning_rate, float learning_rate_value, int32_t clip_mask,
    float min_value, float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream);
int scemb_sparse_dense_matmul_grad_with_adagrad(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, float* accumulator,
    int64_t table_rows, int32_t dim, const float* learning_rate,
    float learning_rate_value, int32_t clip_mask, float min_value,
    float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream);
/* The same two updates reading the activation gradients from per-feature
 * blocks (no stacked gradient matrix); workspace as above. */
int scemb_sparse_dense_matmul_grad_with_sgd_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    int64_t table_rows, int32_t dim, const float* learning_rate,
    float learning_rate_value, int32_t clip_mask, float min_value,
    float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream);
int scemb_sparse_dense_matmul_grad_with_adagrad_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    float* accumulator, int64_t table_rows, int32_t dim,
    const float* learning_rate, float learning_rate_value, int32_t clip_mask,
    float min_value, float max_value, void* workspace, size_t workspace_bytes,
    uint32_t* device_status, void* stream);

/* ---- Backward + any built-in optimizer ----------------------------------
 * The reference lowers every optimizer to the same custom call,
 * SparseDenseMatmulGradOpWithOptimizerUpdate, with num_slot_variables,
 * num_hyperparameters and a row-wise update function
 * (primitives/sparse_dense_matmul_grad_with_{sgd,adagrad,adam,
 * adagrad_momentum,ftrl,laprop,f2a}.py, the `operands` lists of each
 * lowering). These two entry points are that call: `optimizer` names the
 * update, its slot variables (same shape as the table, updated in place) and
 * hyperparameters, in the order of the primitive's operands:
 *   SGD              slots -;  (learning_rate)
 *   ADAGRAD          slots (accumulator);  (learning_rate)
 *   ADAM             slots (momentum, velocity);
 *                    (alpha_t, beta_1, beta_2, epsilon_hat)
 *   ADAGRAD_MOMENTUM slots (accumulator, momentum);
 *                    (learning_rate, momentum, beta2, epsilon, exponent,
 *                     use_nesterov != 0)
 *   FTRL             slots (accumulator, linear);
 *                    (learning_rate, learning_rate_power, l1, l2, beta);
 *                    flag MULTIPLY_LINEAR_BY_LR
 *   LAPROP           slots (mu, nu);  (learning_rate, b1, decay_rate, eps)
 *   F2A              slots (accumulator, local_step);
 *                    (learning_rate, rho, l1, l2, max_lr_multiplier,
 *                     global_step)
 *   CUSTOM           slots and hyperparameters as `program` declares them
 *                    (primitives/sparse_dense_matmul_optimizer_grad.py:
 *                    147-260, CustomOptimizerSpec)
 * Hyperparameter i is read from the device scalar hyperparameter_ptrs[i]
 * when that is not NULL, else hyperparameters[i] is used. The update of each
 * touched row applies the reference's row-wise function in its operation
 * order, then the clipping as above; the gradient sum is the same fixed-order
 * reduction as the calls above. Workspace:
 * scemb_sparse_dense_matmul_grad_workspace_size. */
#define SCEMB_OPTIMIZER_SGD 0
#define SCEMB_OPTIMIZER_ADAGRAD 1
#define SCEMB_OPTIMIZER_ADAM 2
#define SCEMB_OPTIMIZER_ADAGRAD_MOMENTUM 3
#define SCEMB_OPTIMIZER_FTRL 4
#define SCEMB_OPTIMIZER_LAPROP 5
#define SCEMB_OPTIMIZER_F2A 6
#define SCEMB_OPTIMIZER_CUSTOM 7 /* `program` below; slots 0-2 */
#define SCEMB_MAX_HYPERPARAMETERS 8
/* FTRL's multiply_linear_by_learning_rate (a static attribute of the
 * reference primitive, sparse_dense_matmul_grad_with_ftrl.py). */
#define SCEMB_OPTIMIZER_FLAG_MULTIPLY_LINEAR_BY_LR 1u

/* A custom optimizer's row-wise update: CustomOptimizerSpec's function of
 * (gradient, table, *slots, *hyperparameters) returning (table, *slots)
 * (lib/nn/custom_optimizer_lowering.py, lowered to StableHLO by the
 * reference and run by the SparseCore compiler per embedding row), here as
 * a straight-line program applied to every value of each touched row.
 * Registers hold floats; before the first instruction register 0 holds the
 * row's summed gradient, register 1 the table value, registers 2..
 * 1 + num_slots the slot values and the next num_hyperparameters registers
 * the hyperparameters. Instruction i sets register dst[i] to
 * op[i](a[i], b[i], c[i]) (CONST: the value imm[i]; comparisons give 1 or
 * 0, SELECT(a, b, c) is b where a != 0 else c, CLAMP(a, b, c) is
 * min(max(b, a), c)). Afterwards register out[0] is the new table value
 * (the optimizer's clipping then applies) and out[1 + k] the new value of
 * slot k. Arithmetic is float32 with correctly rounded division and square
 * root; EXP, LOG, POW, TANH, LOG1P and EXPM1 are the device library's
 * double-precision functions rounded once to float.
 * The first call with a program compiles it at run time (hiprtc, about a
 * second per program and layout; kept for the process) into the kernels the
 * built-in optimizers run, with the update inlined. The environment variable
 * SCEMB_CUSTOM_UPDATE chooses: "auto" (default: compiled, or interpreted
 * by the library's own kernels when hiprtc is missing or compilation
 * fails), "compile" (fail with SCEMB_ERR_DEVICE instead of interpreting) or
 * "interpret"; any other value is SCEMB_ERR_INVALID_ARGUMENT. Both forms give
 * identical results. */
#define SCEMB_PROGRAM_MAX_OPS 48
#define SCEMB_PROGRAM_MAX_REGISTERS 24
enum {
  SCEMB_OP_CONST = 0, SCEMB_OP_ADD, SCEMB_OP_SUB, SCEMB_OP_MUL, SCEMB_OP_DIV,
  SCEMB_OP_NEG, SCEMB_OP_SQRT, SCEMB_OP_RSQRT, SCEMB_OP_ABS, SCEMB_OP_EXP,
  SCEMB_OP_LOG, SCEMB_OP_POW, SCEMB_OP_MAX, SCEMB_OP_MIN, SCEMB_OP_SIGN,
  SCEMB_OP_TANH, SCEMB_OP_LOG1P, SCEMB_OP_EXPM1, SCEMB_OP_FLOOR,
  SCEMB_OP_CEIL, SCEMB_OP_SELECT, SCEMB_OP_CMP_EQ, SCEMB_OP_CMP_NE,
  SCEMB_OP_CMP_LT, SCEMB_OP_CMP_LE, SCEMB_OP_CMP_GT, SCEMB_OP_CMP_GE,
  SCEMB_OP_CLAMP, SCEMB_OP_AND, SCEMB_OP_OR, SCEMB_OP_NOT, SCEMB_OP_COUNT
};
typedef struct scemb_update_program {
  int32_t num_ops;
  int32_t num_slots;           /* slot variables (0..2) */
  int32_t num_hyperparameters; /* 0..SCEMB_MAX_HYPERPARAMETERS */
  uint8_t op[SCEMB_PROGRAM_MAX_OPS];
  uint8_t dst[SCEMB_PROGRAM_MAX_OPS];
  uint8_t a[SCEMB_PROGRAM_MAX_OPS];
  uint8_t b[SCEMB_PROGRAM_MAX_OPS];
  uint8_t c[SCEMB_PROGRAM_MAX_OPS];
  float imm[SCEMB_PROGRAM_MAX_OPS];
  uint8_t out[3];
  uint8_t reserved;
} scemb_update_program_t;

typedef struct scemb_optimizer {
  int32_t kind;   /* SCEMB_OPTIMIZER_* */
  uint32_t flags; /* SCEMB_OPTIMIZER_FLAG_* */
  float* slots[2];
  const float* hyperparameter_ptrs[SCEMB_MAX_HYPERPARAMETERS];
  float hyperparameters[SCEMB_MAX_HYPERPARAMETERS];
  int32_t clip_mask; /* bit 0: min_value, bit 1: max_value */
  float min_value;
  float max_value;
  /* SCEMB_OPTIMIZER_CUSTOM: the update (copied at the call, not kept) */
  const scemb_update_program_t* program;
} scemb_optimizer_t;

int scemb_sparse_dense_matmul_grad_with_optimizer(
    const scemb_csr_t* csr, const float* activations_grad,
    int64_t device_batch_size, float* table, int64_t table_rows, int32_t dim,
    const scemb_optimizer_t* optimizer, void* workspace,
    size_t workspace_bytes, uint32_t* device_status, void* stream);
int scemb_sparse_dense_matmul_grad_with_optimizer_from_blocks(
    const scemb_csr_t* csr, const scemb_row_block_t* activation_grads,
    int32_t num_blocks, int64_t device_batch_size, float* table,
    int64_t table_rows, int32_t dim, const scemb_optimizer_t* optimizer,
    void* workspace, size_t workspace_bytes, uint32_t* device_status,
    void* stream);

/* ---- Preprocessing: PreprocessSparseDenseMatmulInput, one stacked table --
 * Inputs: the features of one stack, in row_offset order (the order
 * GetStackedTableMetadata produces, pybind_input_preprocessing.cc:114-120).
 * Each feature is values + row splits (or a fixed valency) in device memory;
 * the host copy of the row splits lets the library plan slice offsets
 * without a device read (if it is NULL and the device splits are given, the
 * call reads them back synchronously). */
typedef struct scemb_feature {
  const int32_t* ids;              /* device [nnz] */
  const float* weights;            /* device [nnz] or NULL (unity weights) */
  const int64_t* row_splits;       /* device [num_rows + 1] or NULL */
  const int64_t* row_splits_host;  /* host [num_rows + 1] or NULL */
  int64_t num_rows;
  int64_t nnz;
  int32_t valency;     /* ids per row when row_splits is NULL */
  int32_t row_offset;  /* FeatureIdTransformation.row_offset */
  int32_t col_offset;  /* FeatureIdTransformation.col_offset */
  int32_t col_shift;   /* FeatureIdTransformation.col_shift */
  /* With row_splits: the most ids of one row, or 0 when not known (the
   * library then reads it off the row splits). A hint that picks the
   * grouping route (scemb_preprocess_options_t.flags); any value gives the
   * same outputs. An understated hint costs time, not correctness: a row of
   * more than 896 ids then goes through the route that merges duplicates at
   * extraction, where its duplicate scan runs from global memory and grows
   * with the square of the row length (about 10^10 loads for one row of
   * 10^5 ids). Pass 0 rather than a guess. */
  int64_t max_row_length;
} scemb_feature_t;

/* Checks host row splits [num_rows + 1] (start at 0, non-decreasing, end at
 * nnz; the RaggedTensorInputBatch contract, ragged_tensor_input_batch.h:
 * 68-127) in one pass and returns the most ids of one row in
 * *max_row_length. SCEMB_ERR_INVALID_ARGUMENT when they do not hold. */
int scemb_check_row_splits(const int64_t* row_splits, int64_t num_rows,
                           int64_t nnz, int64_t* max_row_length);

/* scemb_check_row_splits that also copies the splits to host memory dst
 * [num_rows + 1] (a staging buffer for the upload) in the same pass. */
int scemb_stage_row_splits(const int64_t* row_splits, int64_t num_rows,
                           int64_t nnz, int64_t* dst,
                           int64_t* max_row_length);

/* No counterpart in the reference (its row splits never leave the host).
 * scemb_stage_row_splits for `count` features in one call, their rows spread
 * over a few host threads: feature i's splits row_splits[i] [num_rows[i] + 1]
 * are checked against nnz[i], copied to dst[i] and their longest row stored
 * in max_row_length[i]. SCEMB_ERR_INVALID_ARGUMENT when any feature's splits
 * do not hold; *first_bad (may be null) is then its index, else -1. */
int scemb_stage_row_splits_batch(int32_t count,
                                 const int64_t* const* row_splits,
                                 const int64_t* num_rows, const int64_t* nnz,
                                 int64_t* const* dst, int64_t* max_row_length,
                                 int32_t* first_bad);

/* scemb_preprocess_options_t.flags. Where the features' sample rows are
 * disjoint and neither id dropping nor minibatching is on, the library merges
 * the copies of an id within one input row while extracting (the only
 * duplicates such an input can hold) and sorts the distinct entries; a
 * sample view then also needs a static buffer of at least the theoretical
 * size (scemb_compute_theoretical_max_coo_buffer_size). Otherwise it sorts
 * every id and merges duplicates after the sort. Both routes give the same
 * outputs; this flag forces the second, for comparison. */
#define SCEMB_PREPROCESS_GROUP_AFTER_SORT 1

typedef struct scemb_preprocess_options {
  int32_t local_device_count;
  int32_t global_device_count;
  int32_t num_sc_per_device;
  int32_t combiner;  /* 0 sum, 1 mean, 2 sqrtn */
  int32_t max_ids_per_partition;
  int32_t max_unique_ids_per_partition;
  int32_t allow_id_dropping;
  int32_t has_variable_weights; /* weights given for the stack's features */
  int64_t coo_buffer_size_per_device;
  int64_t col_id_bound; /* exclusive bound on column ids (stack vocab size) */
  /* 1: also write the sample view of the CSR (scemb_sample_view_t) into
   * out->view_keys / view_entries, without a sort: the entries come out of
   * the preprocessing already grouped by activation row. Needs
   * local_device_count = global_device_count = 1 and features whose sample
   * rows do not overlap (row_offset order, as GetStackedTableMetadata gives
   * them); entries of one activation row are in input order of their first
   * id (scemb_build_sample_view keeps CSR order instead; both group the same
   * entries). Entries whose embedding id is outside the table (table_rows /
   * num_partitions rows per partition) are left out, as the forward skips
   * them. */
  int32_t build_sample_view;
  /* Minibatching (PreprocessSparseDenseMatmulInputOptions.enable_minibatching,
   * input_preprocessing_util.h:472; single host). One call per pass and
   * stack, in the order of input_preprocessing.cc:852-929:
   *   pass 0  the first pass over every stack: the stats (which stay those of
   *           the call), the CSR of one minibatch, and counter 4 = 1 when a
   *           partition exceeds a limit (no id is dropped in this pass); then
   *           also counter 5 = this stack's split of the 64 buckets, from its
   *           runs counted per bucket (OR it over all stacks);
   *   pass 1  the bucket pass itself, counter 5 = the same split (optional:
   *           pass 0 already gives it);
   *   pass 2  the bucket pass writing popcount(split) + 1 minibatches, with
   *           minibatching_split = that OR; counter 0 = its dropped ids.
   * Row pointers then take 64 * S * max(NS, 8) entries per device (the first
   * S * minibatches * max(NS, 8) written) and hold device positions; the
   * buffer size bound is 64 times larger (scemb_compute_*). */
  int32_t enable_minibatching;
  int64_t table_rows; /* rows of the device's table, for the sample view */
  int32_t minibatching_pass;
  int32_t flags; /* SCEMB_PREPROCESS_* bits; 0 for the default route */
  uint64_t minibatching_split; /* pass 2: bit i set = tree node i split
                                  (MinibatchingSplit, input_preprocessing_
                                  util.h:94) */
} scemb_preprocess_options_t;

/* Device outputs. The stats block is int32 laid out as
 *   [L*NS] max_ids_per_partition, [L*NS] max_unique_ids_per_partition,
 *   [L*S] required_buffer_size, then 6 int64 counters (8-byte aligned by the
 *   caller): dropped_id_count, limit_exceeded, bad_ids, total_entries,
 *   minibatching_required (pass 0), minibatching_split (pass 1). The call
 *   initialises the whole block; the caller need not clear it. */
typedef struct scemb_preprocess_output {
  int32_t* row_pointers;  /* [L * S * max(NS, 8)] (times 64, minibatching) */
  int32_t* embedding_ids; /* [L * coo_buffer_size_per_device] */
  int32_t* sample_ids;    /* [L * coo_buffer_size_per_device] */
  float* gains;           /* [L * coo_buffer_size_per_device] */
  int32_t* stats;         /* scemb_preprocess_stats_size() int32 slots */
  uint32_t* view_keys;     /* [coo_buffer_size_per_device], build_sample_view */
  uint64_t* view_entries;  /* [coo_buffer_size_per_device], build_sample_view */
} scemb_preprocess_output_t;

int64_t scemb_preprocess_stats_size(const scemb_preprocess_options_t* opts);
int64_t scemb_preprocess_stats_counters_offset(
    const scemb_preprocess_options_t* opts);
size_t scemb_preprocess_workspace_size(const scemb_feature_t* features,
                                       int32_t num_features,
                                       const scemb_preprocess_options_t* opts);
int scemb_preprocess_stacked_table(const scemb_feature_t* features,
                                   int32_t num_features,
                                   const scemb_preprocess_options_t* opts,
                                   const scemb_preprocess_output_t* out,
                                   void* workspace, size_t workspace_bytes,
                                   void* stream);

/* Several stacked tables of one batch in one call, as the reference's
 * PreprocessSparseDenseMatmulInput takes them all (input_preprocessing.cc:
 * 827-868 extracts, sorts and groups every table, then fills every table's
 * buffers). Job i is scemb_preprocess_stacked_table's arguments for one
 * stack, with its own workspace of scemb_preprocess_workspace_size() bytes.
 * Each stage of the stacks that merge duplicates at extraction is one launch
 * for all of them (those of one key width and weighting); the others run one
 * after another. The outputs are those of one call per job. */
typedef struct scemb_preprocess_job {
  const scemb_feature_t* features;
  int32_t num_features;
  const scemb_preprocess_options_t* options;
  const scemb_preprocess_output_t* outputs;
  void* workspace;
  size_t workspace_bytes;
} scemb_preprocess_job_t;

int scemb_preprocess_stacked_tables(const scemb_preprocess_job_t* jobs,
                                    int32_t num_jobs, void* stream);

/* ---- Launch timing (no counterpart in the reference) -------------------
 * For benchmarks: while enabled, the library records HIP events on the launch
 * stream around its main kernels ("fwd_reduce", "fwd_finish", "bwd_reduce",
 * "bwd_finish") and around whole calls ("fwd_call", "bwd_call",
 * "preprocess_call").
 * scemb_profile_collect waits for the recorded events of `name` (all names
 * when NULL), returns their summed elapsed milliseconds and launch count,
 * and forgets them. */
void scemb_profile_enable(int enable);
int scemb_profile_collect(const char* name, double* total_ms,
                          int64_t* launches);

/* ---- Size helpers (host only) -----------------------------------------
 * ComputeTheoreticalMaxCooBufferSize (input_preprocessing_util.cc:244-255),
 * ComputeCooBufferSizePerDevice (:256-312; returns -1 when the suggestion
 * exceeds the theoretical maximum), and GetRowPointersSizePerDevice
 * (input_preprocessing_util.h:497-511), as bound with their
 * enable_minibatching argument at pybind_input_preprocessing.cc:218-244. */
int64_t scemb_compute_theoretical_max_coo_buffer_size(
    int32_t max_ids_per_partition, int32_t global_device_count,
    int32_t num_sc_per_device, int32_t enable_minibatching);
int64_t scemb_compute_coo_buffer_size_per_device(
    int32_t max_ids_per_partition, int64_t suggested_coo_buffer_size,
    int32_t global_device_count, int32_t num_sc_per_device,
    int32_t enable_minibatching);
int32_t scemb_compute_row_pointers_size_per_device(int32_t global_device_count,
                                                   int32_t num_sc_per_device,
                                                   int32_t enable_minibatching);

#ifdef __cplusplus
}
#endif

#endif /* SCEMB_H_ */
