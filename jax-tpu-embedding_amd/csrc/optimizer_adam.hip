// Backward segmented reduction fused with the Adam row update
// (lib/core/primitives/sparse_dense_matmul_grad_with_adam.py), in a translation
// unit of its own so that the optimizers compile in parallel.
#include "segreduce.h"

namespace scemb {

int GradWithAdam(const GradCall& c) { return GradImpl<kEpiAdam>(c); }

}  // namespace scemb
