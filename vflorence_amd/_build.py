"""In-tree builds (no cmake): libvflorence_amd.so for gfx950 (hipcc) and the engine's
native host core libvfl_host.so (g++, CPU only).

    python -m vflorence_amd._build          # or __graft_entry__.build()

The libraries are written next to this file so they travel with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
SOURCES = ("kv_cache.hip", "paged_attention.hip", "attention_dims.hip", "attention_block32.hip",
           "decoder_ops.hip", "decode_linear.hip")
OUTPUT = os.path.join(HERE, "libvflorence_amd.so")
ARCH = os.environ.get("VFL_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
# -amdgpu-mfma-vgpr-form: matrix-core results in ordinary VGPRs, so accumulators that the
# online softmax rescales between products are not copied to and from AGPRs around every
# product (the beam-group self-attention kernel lost 144 such moves, 12 VGPRs).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


HOST_SOURCES = ("host/engine_core.cpp",)
HOST_OUTPUT = os.path.join(HERE, "libvfl_host.so")
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror"]


def build_host_library(verbose: bool = False) -> str:
    """Compile the engine's host core into HOST_OUTPUT; always recompiles."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if not cxx:
        raise RuntimeError("g++ not found; the engine's host core cannot be built")
    tmp = HOST_OUTPUT + ".tmp"
    cmd = [cxx, *HOST_FLAGS, *[os.path.join(CSRC, s) for s in HOST_SOURCES], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("g++ failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, HOST_OUTPUT)
    return HOST_OUTPUT


def build_library(verbose: bool = False) -> str:
    """Compile every HIP source into OUTPUT; always recompiles.  The sources compile to
    objects in parallel (one hipcc per file), then link into the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    # The host pass does not know the gfx950 feature flag; that warning is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]

    def compile_one(src: str):
        obj = os.path.join(objdir, os.path.splitext(os.path.basename(src))[0] + ".o")
        cmd = [hipcc(), *flags, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln]
        return obj, proc.returncode, msgs

    workers = max(1, min(len(SOURCES), os.cpu_count() or 1))
    with ThreadPoolExecutor(workers) as pool:
        results = list(pool.map(compile_one, SOURCES))
    for _, rc, msgs in results:
        if rc != 0:
            raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
        if verbose and msgs:
            print("\n".join(msgs), flush=True)
    tmp = OUTPUT + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *[obj for obj, _, _ in results], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
    print(build_host_library(verbose="-v" in sys.argv))
