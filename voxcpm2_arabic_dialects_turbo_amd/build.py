"""Builds libvoxattn.so in-tree with hipcc for gfx950 (run as ``python -m voxcpm2_arabic_dialects_turbo_amd.build``).

The attention library is one shared library, C ABI only (include/vox_attn.h): no torch headers, no pybind. The
sources compile in parallel and link into ``voxcpm2_arabic_dialects_turbo_amd/libvoxattn.so``. Beside it,
``libvoxprobe.so`` (include/vox_probe.h) holds the memory-rate probes bench.py runs; the attention path never loads
it. Packed FP32 VALU instructions are disabled for
device code (``-packed-fp32-ops``); hipcc's host pass warns that it does not know that feature, which is harmless.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libvoxattn.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["store_kvcache.hip", "decode_attn.hip", "prefill_attn.hip", "quantize_rows.hip", "kv_copy.hip", "capi.hip"]
PROBE_PATH = os.path.join(PKG_DIR, "libvoxprobe.so")
PROBE_SOURCES = ["bench_probe.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libvoxattn.so")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-munsafe-fp-atomics",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{os.path.join(REPO_DIR, 'include')}",
        f"-I{CSRC}",
    ]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # the host pass's "not a recognized feature" warnings for -packed-fp32-ops are expected noise
    noise = "'-packed-fp32-ops' is not a recognized feature"
    text = "\n".join(line for line in proc.stdout.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{text}")
    if text.strip():
        print(text, file=sys.stderr)


def build(verbose: bool = False) -> str:
    """Compiles every source and links libvoxattn.so and libvoxprobe.so; returns the attention library's path.
    Always rebuilds."""
    cc = hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    cmds = []
    for src in SOURCES + PROBE_SOURCES:
        obj = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        cmds.append([cc, *compile_flags(), "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            if verbose:
                print(" ".join(cmd))
            fut.result()
    for path, srcs in ((LIB_PATH, SOURCES), (PROBE_PATH, PROBE_SOURCES)):
        objs = [os.path.join(BUILD_DIR, src.replace(".hip", ".o")) for src in srcs]
        tmp = path + ".tmp"
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
        os.replace(tmp, path)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
