// Backward segmented reduction fused with the LaProp row update
// (lib/core/primitives/sparse_dense_matmul_grad_with_laprop.py), in a
// translation unit of its own so that the optimizers compile in parallel.
#include "segreduce.h"

namespace scemb {

int GradWithLaprop(const GradCall& c) { return GradImpl<kEpiLaprop>(c); }

}  // namespace scemb
