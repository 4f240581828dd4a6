// The key-side backward kernel at bf16 head dim 64 for one-head sequences (see sa_bf16_kv.hip),
// built with sa_bf16.hip's flags: its one-head instance (SOLO) holds head 0's tile loop only, 231
// registers without spills under the iterative scheduler (with the other heads' loop built beside
// it, that scheduler spills 63).

#include "sa_kernels.h"

namespace sa_host {

int launch_bwd_kv64_solo(bool cv, const KvLaunch& a) {
  if (cv) launch_kv64_from<true, true>(a);
  else launch_kv64_from<false, true>(a);
  return launch_status();
}

}  // namespace sa_host
