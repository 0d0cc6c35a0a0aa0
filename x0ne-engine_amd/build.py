"""Builds libx0ne_core.so in-tree: every csrc/*.hip compiled for gfx950 by hipcc, then linked.

Flags: -ffp-contract=off (no multiply-add is fused unless the code writes fmaf, so the norms,
RoPE and the weight initialiser round where the oracle rounds) and
`-Xclang -target-feature -Xclang -packed-fp32-ops` (no packed f32 instructions are generated).
The kernel-set fingerprint is the SHA-256 of the sources, compiled into the library.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "x0ne_core", "libx0ne_core.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-parameter",
    "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def fingerprint() -> str:
    h = hashlib.sha256()
    for f in sorted(os.listdir(CSRC)):
        if f.endswith((".hip", ".h")):
            h.update(f.encode())
            with open(os.path.join(CSRC, f), "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


# --asan: the host code (loaders, parsers, arena, runtime) under AddressSanitizer; the device
# code is unchanged. Output x0ne_core/libx0ne_core_asan.so, loaded with the sanitizer runtime
# preloaded and X0NE_CORE_LIB naming it.
ASAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]
ASAN_LIB = os.path.join(HERE, "x0ne_core", "libx0ne_core_asan.so")


def _compile(src: str, kernel_set: str, asan: bool = False) -> str:
    out_dir = OUT_DIR + ("_asan" if asan else "")
    obj = os.path.join(out_dir, src.replace(".hip", ".o"))
    cmd = [HIPCC] + FLAGS + (ASAN_FLAGS if asan else []) + [f'-DX0NE_KERNEL_SET="{kernel_set}"', "-c",
                                                            os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    # The host pass does not know the packed-fp32 feature; that warning is expected.
    noise = [l for l in r.stderr.splitlines() if l.strip() and "packed-fp32-ops" not in l
             and "not a recognized feature" not in l]
    if noise:
        sys.stderr.write(f"[{src}]\n" + "\n".join(noise) + "\n")
    return obj


def build(jobs: int | None = None, asan: bool = False) -> str:
    os.makedirs(OUT_DIR + ("_asan" if asan else ""), exist_ok=True)
    kernel_set = fingerprint()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, kernel_set, asan), sources()))
    lib = ASAN_LIB if asan else LIB
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC"] + (ASAN_FLAGS if asan else []) + ["-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(asan="--asan" in sys.argv[1:]))
