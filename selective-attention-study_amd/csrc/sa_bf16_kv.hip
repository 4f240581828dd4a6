// The key-side backward kernel's bf16-storage instances at head dim 64, in translation units of
// their own, compiled in parallel with the rest. This unit (accumulators in VGPRs, the compiler's
// default scheduler) serves sequences of several heads; sa_bf16_kv1.hip (with sa_bf16.hip's
// iterative scheduler as well) the one-head sequences, whose workgroups all take the head-0 tile
// loop, which that scheduler runs faster (measured: the loop of the other heads runs faster under
// the default one). The other head dims' instances are in sa_bf16_kvg.hip.

#include "sa_kernels.h"

namespace sa_host {

int launch_bwd_kv_bf16(int D, int G, bool cv, const KvLaunch& a) {
  if (D != 64) return launch_bwd_kv_bf16_generic(D, G, cv, a);
  if (a.H == 1) return launch_bwd_kv64_solo(cv, a);
  if (cv) launch_kv64_from<true, false>(a);
  else launch_kv64_from<false, false>(a);
  return launch_status();
}

}  // namespace sa_host
