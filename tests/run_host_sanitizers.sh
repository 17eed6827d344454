#!/bin/bash
# Host-side AddressSanitizer + UndefinedBehaviorSanitizer run of the library's
# argument checks, plans and workspace arithmetic (CPU only; no GPU needed).
# Builds mlx-server-runtime_amd/_build_san/libmi355q_san.so from the same
# sources with the host code instrumented (device code unchanged), then runs
# tests/test_host.py against it with the clang ASan runtime preloaded.
#
#   bash tests/run_host_sanitizers.sh
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
PKG="$ROOT/mlx-server-runtime_amd"
OUT="$PKG/_build_san"
mkdir -p "$OUT"
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
FLAGS="-O1 -g -std=c++17 -fPIC --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops -I $ROOT/include"
export HIPCC FLAGS OUT
ls "$PKG"/csrc/*.hip | xargs -P 8 -I{} bash -c '"$HIPCC" $FLAGS -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=all -Xarch_host -fno-omit-frame-pointer -c "$1" -o "$OUT/$(basename "$1").o" 2>&1 | grep -v "packed-fp32-ops. is not a recognized feature" || true' _ {}
"$HIPCC" -shared -fPIC --offload-arch=gfx950 -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -shared-libasan "$OUT"/*.o -o "$OUT/libmi355q_san.so"
ASAN_RT=$("$HIPCC" -print-file-name=libclang_rt.asan-x86_64.so)
echo "sanitized library: $OUT/libmi355q_san.so; runtime: $ASAN_RT"
cd "$ROOT"
LD_PRELOAD="$ASAN_RT" MQ_LIBRARY_PATH="$OUT/libmi355q_san.so" \
  ASAN_OPTIONS=detect_leaks=0:halt_on_error=1:abort_on_error=1 \
  UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \
  python -m pytest tests/test_host.py -q -p no:cacheprovider
