"""Builds libmsx.so (host runtime + gfx950 kernels, one hipcc invocation) in-tree.

The shared library is the product: the C ABI of include/msx.h over the HIP runtime. Every
source is compiled with -ffp-contract=off (no fusion the source does not write) and the packed
FP32 instructions disabled; kernels target gfx950 only.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmsx.so")
CODE_OBJECTS = os.path.join(HERE, "kernels")
SOURCES = [
    "capi.cpp",
    "host/ir.cpp",
    "host/passes.cpp",
    "host/rng.cpp",
    "host/models.cpp",
    "host/mspec.cpp",
    "host/runner.cpp",
    "host/json.cpp",
    "host/packed.cpp",
    "host/checkpoint.cpp",
    "host/artifact.cpp",
    "hip/runtime.cpp",
    "hip/kernels.hip",
    "hip/gemm.hip",
    "hip/gemm_lds.hip",
    "hip/attention.hip",
    "hip/flash16.hip",
    "hip/data.hip",
    "hip/segments.hip",
]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-std=c++17", "-O3", "-fPIC", "-shared", "--offload-arch=gfx950",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-parameter", "-Wno-unused-result",
]


# Per-source flags. The direct-to-LDS GEMMs and the f16 attention keep their MFMA accumulators in VGPRs: with the
# compiler's default choice (AGPRs) it rotated the accumulators through copies every K tile.
FILE_FLAGS = {"hip/gemm_lds.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              "hip/flash16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def build(verbose=False):
    objs = []
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    procs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        obj = os.path.join(build_dir, src.replace("/", "_") + ".o")
        lang = ["-x", "hip"] if src.endswith((".hip", "runtime.cpp", "capi.cpp")) else []
        cmd = [HIPCC] + [f for f in FLAGS if f != "-shared"] + FILE_FLAGS.get(src, []) + ["-c"] + lang + [path, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
    # The gfx950 code object of each kernel source, beside the library: what an artifact of the
    # library's plans records and hashes (host/artifact.cpp).
    os.makedirs(CODE_OBJECTS, exist_ok=True)
    for src in SOURCES:
        if not src.endswith(".hip"):
            continue
        out = os.path.join(CODE_OBJECTS, os.path.basename(src).replace(".hip", ".hsaco"))
        cmd = ([HIPCC] + [f for f in FLAGS if f not in ("-shared", "-fPIC")] + FILE_FLAGS.get(src, []) +
               ["--genco", "--offload-device-only", "--no-gpu-bundle-output", os.path.join(CSRC, src), "-o", out])
        procs.append((src + " (code object)", subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        if p.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        for src, text in failed:
            sys.stderr.write(f"--- {src}\n{text}\n")
        raise RuntimeError("hipcc failed for " + ", ".join(s for s, _ in failed))
    # Linked beside the library and renamed over it, so a process that has the old one mapped
    # keeps its pages.
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC] + FLAGS + objs + ["-o", tmp], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
