#!/usr/bin/env bash
# Builds libsa_hip.so (gfx950) next to the Python package. Run from anywhere; extra arguments are
# passed to every compile (e.g. -DSA_FWD_MIN_BLOCKS=2). SA_OUT overrides the output path.
#
# Translation units, compiled in parallel:
#   sa_bf16.hip  bf16-storage kernels, -amdgpu-mfma-vgpr-form: MFMA accumulators in VGPRs (left to
#                its heuristics the compiler keeps them in AGPRs and copies every loop-carried
#                accumulator back and forth each iteration), and the compiler's iterative ILP
#                scheduler (faster for the tile loops than the default one)
#   sa_bf16_kv.hip  the bf16 key-side backward kernel at head dim 64 for sequences of several
#                heads: accumulators in VGPRs, the default scheduler (2% faster there than the
#                iterative one)
#   sa_bf16_kv1.hip  the same kernel for one-head sequences (every workgroup in the head-0 loop),
#                sa_bf16.hip's flags (4% faster there)
#   sa_bf16_kvg.hip  the bf16 key-side instances at head dims 32 and 128: accumulators in VGPRs,
#                the default scheduler (the two options together crash this compiler on them)
#   sa_bf16_dec.hip  the bf16 decode-step kernels, the default scheduler (faster for them)
#   sa_f32.hip   fp32-storage kernels, the compiler's own accumulator placement
#   sa_abi.hip   the C ABI (host code only)
# Every HIP compile: -packed-fp32-ops off (no v_pk_*_f32 from the compiler).
set -euo pipefail
here="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
root="$(cd "$here/../.." && pwd)"
out="${SA_OUT:-$here/../selective_attention/libsa_hip.so}"
tmp="$(mktemp -d)"
trap 'rm -rf "$tmp"' EXIT

common=(--offload-arch=gfx950 -O3 -std=c++17 -fPIC -munsafe-fp-atomics
        -Xclang -target-feature -Xclang -packed-fp32-ops -I"$root/include" "$@")

# unit <source> <object> [compiler-internal options...]: the options (-mllvm ...) are this compiler's
# internal knobs, not a stable interface; if a compiler release drops or rejects them the unit is
# compiled again without them (correct code, slower tile loops) and the build says so.
unit() {
  local src=$1 obj=$2
  shift 2
  if hipcc "${common[@]}" "$@" -c "$here/$src" -o "$tmp/$obj" 2> "$tmp/$obj.err"; then
    grep -v "packed-fp32-ops" "$tmp/$obj.err" >&2 || true
    return 0
  fi
  if [ $# -eq 0 ]; then cat "$tmp/$obj.err" >&2; return 1; fi
  echo "build.sh: $src failed with the internal options ($*); compiling it without them" >&2
  hipcc "${common[@]}" -c "$here/$src" -o "$tmp/$obj"
}

tuned=(-mllvm -amdgpu-mfma-vgpr-form -mllvm -amdgpu-sched-strategy=iterative-ilp)
unit sa_bf16.hip sa_bf16.o "${tuned[@]}" &
p1=$!
unit sa_bf16_kv.hip sa_bf16_kv.o -mllvm -amdgpu-mfma-vgpr-form &
p4=$!
unit sa_bf16_kv1.hip sa_bf16_kv1.o "${tuned[@]}" &
p7=$!
unit sa_bf16_kvg.hip sa_bf16_kvg.o -mllvm -amdgpu-mfma-vgpr-form &
p6=$!
unit sa_bf16_dec.hip sa_bf16_dec.o -mllvm -amdgpu-mfma-vgpr-form &
p5=$!
unit sa_f32.hip sa_f32.o &
p2=$!
unit sa_abi.hip sa_abi.o &
p3=$!
rc=0
wait $p1 || rc=1
wait $p2 || rc=1
wait $p3 || rc=1
wait $p4 || rc=1
wait $p5 || rc=1
wait $p6 || rc=1
wait $p7 || rc=1
[ $rc -eq 0 ] || { echo "build.sh: a compile failed" >&2; exit 1; }
hipcc --offload-arch=gfx950 -shared -fPIC "$tmp/sa_bf16.o" "$tmp/sa_bf16_kv.o" "$tmp/sa_bf16_kv1.o" "$tmp/sa_bf16_kvg.o" "$tmp/sa_bf16_dec.o" "$tmp/sa_f32.o" \
  "$tmp/sa_abi.o" \
  -o "$out.tmp"
mv "$out.tmp" "$out"
echo "built $out"
