// Backward segmented reduction fused with the Adagrad-with-momentum row update
// (lib/core/primitives/sparse_dense_matmul_grad_with_adagrad_momentum.py), in a
// translation unit of its own so that the optimizers compile in parallel.
#include "segreduce.h"

namespace scemb {

int GradWithAdagradMomentum(const GradCall& c) {
  return GradImpl<kEpiAdagradMomentum>(c);
}

}  // namespace scemb
