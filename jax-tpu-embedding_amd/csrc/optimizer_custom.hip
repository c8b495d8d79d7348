// Backward segmented reduction fused with a custom optimizer's row update
// (CustomOptimizerSpec, lib/core/primitives/sparse_dense_matmul_optimizer_grad.py):
// the update is a straight-line program interpreted per table value
// (RunProgram in segreduce.h). Programs of arithmetic operations only run
// here; those using a transcendental operation run the kernels of
// optimizer_custom_transcendental.hip.
#include "segreduce.h"

namespace scemb {

int GradWithCustom(const GradCall& c) {
  if (c.opt.prog.transcendental) return GradWithCustomTranscendental(c);
  return GradImpl<kEpiCustomArith>(c);
}

}  // namespace scemb
