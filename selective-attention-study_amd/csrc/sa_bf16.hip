// The kernels' bf16-storage instances (bf16 MFMA operands, fp32 accumulation). Built with the MFMA
// accumulators held in VGPRs (build.sh): left to its heuristics the compiler keeps them in AGPRs
// and copies every loop-carried accumulator back and forth each iteration.

#include "sa_kernels.h"

namespace sa_host {

int forward_bf16(const FwdCall& c) { return forward_entry<OpBF16>(c); }
int backward_bf16(const BwdCall& c) { return backward_entry<OpBF16>(c); }

}  // namespace sa_host
