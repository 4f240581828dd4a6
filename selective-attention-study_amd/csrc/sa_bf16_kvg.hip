// The key-side backward kernel's bf16-storage instances at head dims 32 and 128 (the generic
// kernel), in a translation unit of their own: built with the MFMA accumulators in VGPRs but the
// compiler's default scheduler (with both of sa_bf16.hip's options this compiler crashes on them).

#include "sa_kernels.h"

namespace sa_host {

int launch_bwd_kv_bf16_generic(int D, int G, bool cv, const KvLaunch& a) {
#define SA_KV(DD, GG)                                        \
  if (cv) launch_kv_from<OpBF16, DD, GG, true>(a);           \
  else launch_kv_from<OpBF16, DD, GG, false>(a);             \
  return launch_status()
  if (D == 32) {
    if (G == 2) { SA_KV(32, 2); }
    SA_KV(32, 1);
  }
  SA_KV(128, 1);
#undef SA_KV
}

}  // namespace sa_host
