#!/bin/bash
# Host-side AddressSanitizer + UndefinedBehaviorSanitizer run of libnqamd's C ABI
# (argument checks and launch planning; abi_checks.cpp). CPU only: the driver
# exits without running anything where a GPU is visible. The sanitizers apply
# to host code only (-Xarch_host); device code is built as for the library.
# Usage: bash tests/host_sanitizer/build_and_run.sh [work dir, default /tmp/nq_host_san]
set -euo pipefail
here=$(cd "$(dirname "$0")" && pwd)
repo=$(cd "$here/../.." && pwd)
work=${1:-/tmp/nq_host_san}
mkdir -p "$work/obj"
hipcc=${HIPCC:-/opt/rocm/bin/hipcc}
san=(-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=undefined
     -Xarch_host -fno-omit-frame-pointer)
for src in "$repo"/nanoquant_amd/csrc/*.hip; do
  "$hipcc" --offload-arch=gfx950 -O3 -g -Xarch_host -O1 -std=c++17 -fPIC -I"$repo/include" \
    -Xclang -target-feature -Xclang -packed-fp32-ops "${san[@]}" \
    -c "$src" -o "$work/obj/$(basename "$src" .hip).o" &
done
wait
"$hipcc" --offload-arch=gfx950 -shared -fPIC "${san[@]}" -Xarch_host -shared-libasan "$work"/obj/*.o \
  -o "$work/libnqamd_san.so"
/opt/rocm/llvm/bin/clang++ -O1 -g -std=c++17 -fsanitize=address,undefined -fno-sanitize-recover=undefined \
  -shared-libasan -I"$repo/include" -I/opt/rocm/include -D__HIP_PLATFORM_AMD__ "$here/abi_checks.cpp" \
  -L"$work" -lnqamd_san -L/opt/rocm/lib -lamdhip64 -Wl,-rpath,"$work" -Wl,-rpath,/opt/rocm/lib \
  -o "$work/abi_checks"
asan_rt=$(/opt/rocm/llvm/bin/clang++ -print-file-name=libclang_rt.asan-x86_64.so)
ASAN_OPTIONS=detect_leaks=0:abort_on_error=1 UBSAN_OPTIONS=print_stacktrace=1 LD_PRELOAD="$asan_rt" \
  "$work/abi_checks"
