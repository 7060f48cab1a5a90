#!/usr/bin/env bash
# Builds oracle/_ref/libcwlb_ref.so: the reference's own pure-C++17 host
# functions for this path, compiled from the sources where they lie under
# /root/reference.  Test infrastructure only: its results pin the oracle.
#
# What is compiled, by line range (nothing else of the reference builds here:
# its kernels need a SYCL compiler, its reorder needs oneDPL/TBB and its
# headers pull in Eigen; none of those exist in this image):
#   include/utils.h:15-33     ParallelDataWeighted, SpmmCostParams
#   include/Matrix.h:29-36    CSR_Order
#   src/utils.cpp:832-1021    costWeightedTaskPartitioning
#   src/utils.cpp:1024-1092   save_costs_one_per_line / read_costs_one_per_line
#   main.cpp:86-167           recommended_candidate_w, candidate_search_*
#   main.cpp:281-321          capacity_from_s, wave_based_s
# The translation unit is assembled in a temporary directory outside the
# repository and deleted afterwards; only the .so lands in oracle/_ref/.
# The flags keep IEEE double semantics (no FMA contraction, no fast-math),
# as a generic x86-64 build of the reference has.
set -euo pipefail
REF=${CWLB_REFERENCE_DIR:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
OUT="$HERE/_ref/libcwlb_ref.so"
if [ ! -f "$REF/src/utils.cpp" ]; then
  echo "ref_build: $REF not present; skipping (prebuilt $OUT is used if present)"
  exit 0
fi
mkdir -p "$HERE/_ref"
TMP=$(mktemp -d /tmp/cwlb_ref.XXXXXX)
trap 'rm -rf "$TMP"' EXIT

expect() {  # file line pattern : fail loudly if the reference moved
  if ! sed -n "$2p" "$1" | grep -q -- "$3"; then
    echo "ref_build: $1:$2 does not contain '$3' (reference changed?)" >&2
    exit 1
  fi
}
expect "$REF/include/utils.h" 15 "struct ParallelDataWeighted"
expect "$REF/include/utils.h" 33 "};"
expect "$REF/include/Matrix.h" 29 "class CSR_Order"
expect "$REF/src/utils.cpp" 832 "costWeightedTaskPartitioning"
expect "$REF/src/utils.cpp" 1021 "^}"
expect "$REF/src/utils.cpp" 1024 "bool save_costs_one_per_line"
expect "$REF/src/utils.cpp" 1092 "^}"
expect "$REF/main.cpp" 87 "recommended_candidate_w"
expect "$REF/main.cpp" 167 "^}"
expect "$REF/main.cpp" 281 "double capacity_from_s"
expect "$REF/main.cpp" 321 "^}"

TU="$TMP/ref_tu.cpp"
{
  cat <<'EOF'
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <limits>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>
using namespace std;
EOF
  sed -n 15,33p "$REF/include/utils.h"
  sed -n 29,36p "$REF/include/Matrix.h"
  sed -n 832,1021p "$REF/src/utils.cpp"
  sed -n 1024,1092p "$REF/src/utils.cpp"
  sed -n 86,167p "$REF/main.cpp"
  sed -n 281,321p "$REF/main.cpp"
  cat "$HERE/ref_shim.inc"
} > "$TU"

g++ -std=c++17 -O2 -ffp-contract=off -fno-fast-math -fPIC -shared "$TU" -o "$OUT.tmp"
mv "$OUT.tmp" "$OUT"
echo "ref_build: wrote $OUT"
