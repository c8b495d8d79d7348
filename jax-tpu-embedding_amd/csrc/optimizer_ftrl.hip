// Backward segmented reduction fused with the FTRL row update
// (lib/core/primitives/sparse_dense_matmul_grad_with_ftrl.py), in a translation
// unit of its own so that the optimizers compile in parallel.
#include "segreduce.h"

namespace scemb {

int GradWithFtrl(const GradCall& c) { return GradImpl<kEpiFtrl>(c); }

}  // namespace scemb
