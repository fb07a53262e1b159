#!/bin/bash
# Builds tests/cpp/attn_test against the in-tree libkiln_attn.so (run from anywhere).
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
/opt/rocm/bin/hipcc -O2 -std=c++17 --offload-arch=gfx950 "$HERE/attn_test.cpp" -o "$HERE/attn_test" \
  -L"$ROOT/kiln_amd" -lkiln_attn -Wl,-rpath,"\$ORIGIN/../../kiln_amd"
/opt/rocm/bin/hipcc -O2 -std=c++17 --offload-arch=gfx950 "$HERE/dit_section_test.cpp" -o "$HERE/dit_section_test" \
  -L"$ROOT/kiln_amd" -lkiln_attn -Wl,-rpath,"\$ORIGIN/../../kiln_amd"
