// Custom optimizer updates whose program uses exp, log, pow, tanh, log1p or
// expm1 (evaluated in double precision, inlined): the 4-byte layout only,
// which keeps these kernels free of scratch memory.
#include "segreduce.h"

namespace scemb {

int GradWithCustomTranscendental(const GradCall& c) {
  return GradImpl<kEpiCustom>(c);
}

}  // namespace scemb
