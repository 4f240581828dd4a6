// The key-side backward kernel at bf16 head dim 64 for one-head sequences (see sa_bf16_kv.hip),
// built with sa_bf16.hip's flags.

#include "sa_kernels.h"

namespace sa_host {

int launch_bwd_kv64_solo(bool cv, const KvLaunch& a) {
  if (cv) launch_kv64_from<true>(a);
  else launch_kv64_from<false>(a);
  return launch_status();
}

}  // namespace sa_host
