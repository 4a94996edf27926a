#!/bin/bash
# Host AddressSanitizer + UndefinedBehaviorSanitizer run of the CPU test suite.
#
# Builds, in a scratch copy of the tree (default /tmp/w4a16_sanitize), the host side
# of every native component with -fsanitize=address,undefined:
#   libw4a16.so  -- the C ABI's validation, workspace sizing and dispatch (device code
#                   is compiled as usual: the sanitizer flags are host-only),
#   w4lin_tool   -- the C++ host mirror, its safetensors/JSON parser and census,
#   liboracle_w4a16.so -- the C oracle (built with clang so that one ASan runtime
#                   serves the whole process),
# then runs `pytest -m "not gpu"` there with the ASan runtime preloaded into Python.
# Any sanitizer report aborts the run (halt_on_error), so a green run means none fired.
# Leak detection is off: the Python interpreter does not free everything at exit.
# CPU only: nothing here touches a GPU.
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/.." && pwd)
OUT=${1:-/tmp/w4a16_sanitize}
LLVM=/opt/rocm/llvm
SAN="-fsanitize=address -fsanitize=undefined -fno-sanitize-recover=all -fno-omit-frame-pointer -g"
HOST_SAN="-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=all -Xarch_host -fno-omit-frame-pointer -g"

rm -rf "$OUT"
mkdir -p "$OUT"
(cd "$ROOT" && tar --exclude='*.so' --exclude='./gemma4-zml-probe_amd/w4lin_tool' --exclude='./gemma4-zml-probe_amd/_build' \
    --exclude='__pycache__' -cf - __graft_entry__.py include oracle tests gemma4-zml-probe_amd) | tar -C "$OUT" -xf -

echo "[sanitize] libw4a16.so (host code instrumented)"
make -s -j8 -C "$OUT/gemma4-zml-probe_amd/csrc" \
    HIPFLAGS="-O1 -std=c++17 -fPIC --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops -Wno-unused-command-line-argument $HOST_SAN" \
    LDFLAGS="$HOST_SAN -shared-libsan"
echo "[sanitize] w4lin_tool"
make -s -C "$OUT/gemma4-zml-probe_amd/host" CXXFLAGS="-O1 -std=c++17 -fPIC $HOST_SAN -shared-libsan"
echo "[sanitize] liboracle_w4a16.so (clang)"
make -s -C "$OUT/oracle" CC="$LLVM/bin/clang" CFLAGS="-O1 -fPIC -fopenmp -ffp-contract=off -std=c11 $SAN -shared-libsan"

for f in gemma4-zml-probe_amd/libw4a16.so gemma4-zml-probe_amd/w4lin_tool oracle/liboracle_w4a16.so; do
  nm -D "$OUT/$f" | grep -q __asan_report || { echo "[sanitize] $f is not instrumented" >&2; exit 1; }
done
RT=$("$LLVM/bin/clang" -print-file-name=libclang_rt.asan-x86_64.so)
echo "[sanitize] pytest -m 'not gpu' with $RT"
cd "$OUT"
W4A16_SANITIZER_RUN=1 LD_PRELOAD="$RT" LD_LIBRARY_PATH="$(dirname "$RT"):$LLVM/lib:${LD_LIBRARY_PATH:-}" \
ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1:detect_odr_violation=0:allocator_may_return_null=1:log_path=$OUT/sanitizer" \
UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:log_path=$OUT/sanitizer" \
    python -m pytest tests -q -m "not gpu" -p no:cacheprovider "${@:2}" || rc=$?
# reports go to files (pytest captures the test processes' stderr)
if compgen -G "$OUT/sanitizer*" > /dev/null; then
  cat "$OUT"/sanitizer* >&2
  exit 1
fi
exit "${rc:-0}"
