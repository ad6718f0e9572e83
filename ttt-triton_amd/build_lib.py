"""Build libttt_amd.so (HIP kernels + C ABI) for gfx950 with hipcc.

    python ttt-triton_amd/build_lib.py [-v] [--asan]

Each .hip under csrc/ is compiled to an object in parallel, then linked into
ttt_amd/libttt_amd.so next to the Python loader.  Always rebuilds.

--asan builds a checking copy instead, _build_asan/libttt_amd_asan.so, with
AddressSanitizer on the host code only (the C ABI's validation, size helpers
and launch set-up; device code is built as usual).  Load it with the ASan
runtime preloaded, e.g. for the ABI tests on a machine without a GPU:

    LD_PRELOAD=$(hipcc -print-file-name=libclang_rt.asan-x86_64.so) \
    ASAN_OPTIONS=detect_leaks=0 TTT_AMD_LIB=ttt-triton_amd/_build_asan/libttt_amd_asan.so \
    python -m pytest tests/test_abi.py -m "not gpu"
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "ttt_amd")
LIB = os.path.join(OUT_DIR, "libttt_amd.so")
BUILD_DIR = os.path.join(HERE, "_build")

ARCH = os.environ.get("TTT_AMD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # never emit packed fp32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# per-file additions: the row-split Linear forward keeps its MFMA accumulators
# in VGPRs (its state wave converts W into operand frags every mini-batch)
PER_FILE = {
    "ttt_linear_fwd_rows.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


ASAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
ASAN_DIR = os.path.join(HERE, "_build_asan")


def _compile(src: str, verbose: bool, asan: bool = False) -> str:
    obj = os.path.join(ASAN_DIR if asan else BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *COMMON, *PER_FILE.get(os.path.basename(src), []), *(ASAN if asan else []), "-c", src, "-o", obj]
    if verbose:
        cmd.insert(1, "-Rpass-analysis=kernel-resource-usage")
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(ln for ln in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if verbose and msg.strip():
        print(msg)
    return obj


def build(verbose: bool = False, asan: bool = False) -> str:
    out_dir = ASAN_DIR if asan else BUILD_DIR
    lib = os.path.join(ASAN_DIR, "libttt_amd_asan.so") if asan else LIB
    os.makedirs(out_dir, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, asan), srcs))
    tmp = lib + ".tmp"
    link = ["-Xarch_host", "-fsanitize=address", "-shared-libasan"] if asan else []
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *link, "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, asan="--asan" in sys.argv)
    print(path)
