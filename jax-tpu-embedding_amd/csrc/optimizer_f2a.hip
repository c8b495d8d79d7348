// Backward segmented reduction fused with the frequency-aware Adagrad (F2A) row
// update (lib/core/primitives/sparse_dense_matmul_grad_with_f2a.py), in a
// translation unit of its own so that the optimizers compile in parallel.
#include "segreduce.h"

namespace scemb {

int GradWithF2a(const GradCall& c) { return GradImpl<kEpiF2a>(c); }

}  // namespace scemb
