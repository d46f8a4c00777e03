"""Build recipe for the gfx950 shared library (hipcc, in-tree).

    python -m dan_amd._build          # -> dan_amd/_lib/libdan_tree_attn.so

Flags:
  --offload-arch=gfx950            CDNA4 only, no other targets.
  -mcode-object-version=5          accepted by every ROCm 6/7 runtime (torch
                                   ships its own HIP runtime).
  -target-feature -packed-fp32-ops no packed fp32 VALU instructions.
  -amdgpu-mfma-vgpr-form           matrix-core results in VGPRs, so the softmax
                                   reads the score tile without AGPR copies
                                   (every source but fp8_gemm.hip, whose
                                   accumulators fill the AGPRs).
  -fno-honor-nans -mno-amdgpu-ieee tree_attn.hip only: v_max_f32 without a
                                   canonicalizing max in front of every operand
                                   (the attention's running-max raise). The
                                   other sources keep IEEE NaN semantics, and
                                   host-side argument checks read float bits.

Each source compiles to its own object with its own flags; one link makes
the library.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRCS = [os.path.join(HERE, "csrc", f) for f in ("tree_attn.hip", "qkv_front.hip", "tree_plan.hip", "fp8_quant.hip", "fp8_gemm.hip",
                                                 "gdn.hip", "gdn_chunk.hip", "gdn_conv.hip")]
# Extra flags per source (file name -> flags).
SRC_FLAGS = {"tree_attn.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"]}
# Matrix-core results in VGPRs, for every source but the GEMM, whose 256
# accumulators per lane live in the accumulation registers (AGPRs).
MFMA_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
ACC_IN_AGPRS = {"fp8_gemm.hip"}
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(HERE, "_lib")
OUT = os.path.join(OUT_DIR, "libdan_tree_attn.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 library)")
    return path


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = "is not a recognized feature for this target"
    diag = "\n".join(line for line in (res.stderr or "").splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{diag}")
    if diag.strip() and verbose:
        print(diag, file=sys.stderr)


def build(out=OUT, extra=(), verbose=False):
    """Compile the library; always recompiles. Returns the output path."""
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(os.path.dirname(out), exist_ok=True)
    obj_dir = os.path.join(os.path.dirname(out), "_obj")
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, os.path.basename(src) + ".o") for src in SRCS]
    def flags(src):
        name = os.path.basename(src)
        return [*HIPCC_FLAGS, *([] if name in ACC_IN_AGPRS else MFMA_VGPR_FORM), *SRC_FLAGS.get(name, [])]

    cmds = [[hipcc(), *flags(src), *extra, "-I", INCLUDE, "-c", src, "-o", obj] for src, obj in zip(SRCS, objs)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), max(1, (os.cpu_count() or 1)))) as pool:
        for f in [pool.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = out + ".tmp"
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
