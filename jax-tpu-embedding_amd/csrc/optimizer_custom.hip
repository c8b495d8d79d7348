// Backward segmented reduction fused with a custom optimizer's row update
// (CustomOptimizerSpec, lib/core/primitives/sparse_dense_matmul_optimizer_grad.py):
// the update is a straight-line program interpreted per table value
// (RunProgram in segreduce.h).
#include "segreduce.h"

namespace scemb {

int GradWithCustom(const GradCall& c) { return GradImpl<kEpiCustom>(c); }

}  // namespace scemb
