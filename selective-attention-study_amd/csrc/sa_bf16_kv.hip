// The key-side backward kernel's bf16-storage instances, in a translation unit of their own (built
// with the flags of sa_bf16.hip, in parallel with it).

#include "sa_kernels.h"

namespace sa_host {

int launch_bwd_kv_bf16(int D, int G, bool cv, const KvLaunch& a) {
#define SA_KV(DD, GG)                                        \
  if (cv) launch_kv_from<OpBF16, DD, GG, true>(a);           \
  else launch_kv_from<OpBF16, DD, GG, false>(a);             \
  return launch_status()
  if (D == 32) {
    if (G == 2) { SA_KV(32, 2); }
    SA_KV(32, 1);
  }
  if (D == 64) {   // one head per wavefront at head dim 64: the pipelined kernel
    if (cv) launch_kv64_from<true>(a);
    else launch_kv64_from<false>(a);
    return launch_status();
  }
  SA_KV(128, 1);
#undef SA_KV
}

}  // namespace sa_host
