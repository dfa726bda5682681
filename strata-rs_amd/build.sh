#!/bin/bash
# builds libstrata_hip variants for timing probes
set -e
cd "$(dirname "$0")"
F="--offload-arch=gfx950 -O3 -std=c++17 -fPIC -Xclang -target-feature -Xclang -packed-fp32-ops -I../../include"
for v in base SKIP_APPLY SKIP_LOAD; do
  D=""; [ $v != base ] && D="-D$v"
  mkdir -p o_$v
  for f in api dequant gemv expert moe matmul; do /opt/rocm/bin/hipcc $F $D -c $f.hip -o o_$v/$f.o 2>/dev/null & done; wait
  /opt/rocm/bin/hipcc --offload-arch=gfx950 -shared -fPIC -o lib_$v.so o_$v/*.o
done
