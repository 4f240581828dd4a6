// The cached decode step's bf16-storage kernels, in a translation unit of their own: build.sh
// compiles it with the compiler's default scheduler, which measures faster for these HBM-bound
// kernels than the iterative ILP one the tile loops of sa_bf16.hip use.

#include "sa_kernels.h"

namespace sa_host {

int decode_bf16(const DecCall& c) { return decode_entry<OpBF16>(c); }

}  // namespace sa_host
