#!/bin/bash
# Host sanitizer runs (CPU only, no GPU): the oracle under ASan+UBSan and under TSan, and
# the library's safetensors reader/writer (host code) under ASan+UBSan, with drivers that
# exercise them on valid and malformed input. Run from anywhere: bash tests/sanitize/run.sh
set -euo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
REPO="$(cd "$HERE/../.." && pwd)"
OUT="$HERE/_build"
mkdir -p "$OUT"
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}

echo "[sanitize] oracle, ASan + UBSan"
gcc -O1 -g -std=c11 -pthread -ffp-contract=off -fno-omit-frame-pointer -fsanitize=address,undefined \
    -fno-sanitize-recover=undefined "$HERE/oracle_driver.c" "$REPO/oracle/kt_oracle.c" \
    "$REPO/oracle/kt_oracle_decoder.c" -o "$OUT/oracle_asan" -lm
"$OUT/oracle_asan"

echo "[sanitize] oracle, TSan"
gcc -O1 -g -std=c11 -pthread -ffp-contract=off -fsanitize=thread "$HERE/oracle_driver.c" \
    "$REPO/oracle/kt_oracle.c" "$REPO/oracle/kt_oracle_decoder.c" -o "$OUT/oracle_tsan" -lm
TSAN_OPTIONS=halt_on_error=1 "$OUT/oracle_tsan"

echo "[sanitize] library host code (safetensors reader/writer), ASan + UBSan"
SAN="-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-omit-frame-pointer"
objs=()
for src in "$REPO"/kotensor_amd/csrc/*.hip; do
    obj="$OUT/$(basename "${src%.hip}").o"
    extra=""
    [ "$(basename "$src")" = "kt_quantize.hip" ] && extra="-ffp-contract=off"
    $HIPCC --offload-arch=gfx950 -O1 -g -std=c++17 -fPIC -fno-gpu-flush-denormals-to-zero \
        -Xclang -target-feature -Xclang -packed-fp32-ops $extra $SAN -c "$src" -o "$obj" &
    objs+=("$obj")
done
wait
$HIPCC --offload-arch=gfx950 -shared -fsanitize=address,undefined "${objs[@]}" -o "$OUT/libkotensor_hip_asan.so"
$HIPCC -x c++ -O1 -g -std=c++17 -fsanitize=address,undefined -fno-omit-frame-pointer "$HERE/st_driver.cpp" \
    -x none "$OUT/libkotensor_hip_asan.so" -Wl,-rpath,"$OUT" -o "$OUT/st_asan"
tmp="$(mktemp -d)"
ASAN_OPTIONS=detect_leaks=0 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 "$OUT/st_asan" "$tmp"
rm -rf "$tmp"
echo "[sanitize] all clean"
