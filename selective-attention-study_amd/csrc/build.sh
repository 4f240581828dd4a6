#!/usr/bin/env bash
# Builds libsa_hip.so (gfx950) next to the Python package. Run from anywhere.
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
root="$(cd "$here/../.." && pwd)"
out="${SA_OUT:-$here/../selective_attention/libsa_hip.so}"
# -amdgpu-mfma-vgpr-form: MFMA accumulators live in VGPRs; left to its heuristics the compiler keeps
# them in AGPRs and copies every loop-carried accumulator back and forth each iteration.
hipcc --offload-arch=gfx950 -O3 -std=c++17 -fPIC -shared -munsafe-fp-atomics \
  -Xclang -target-feature -Xclang -packed-fp32-ops -mllvm -amdgpu-mfma-vgpr-form \
  "$@" -I"$root/include" "$here/sa_kernels.hip" -o "$out.tmp"
mv "$out.tmp" "$out"
echo "built $out"
