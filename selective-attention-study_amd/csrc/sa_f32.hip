// The kernels' fp32-storage instances (fp32 MFMA). Built with the compiler's own accumulator
// placement (build.sh): the forced-VGPR form that suits the bf16 instances is beyond this
// compiler's AGPR rewrite pass for the fp32 head-dim-128 backward.

#include "sa_kernels.h"

namespace sa_host {

int forward_f32(const FwdCall& c) { return forward_entry<OpF32>(c); }
int backward_f32(const BwdCall& c) { return backward_entry<OpF32>(c); }
int decode_f32(const DecCall& c) { return decode_entry<OpF32>(c); }

}  // namespace sa_host
