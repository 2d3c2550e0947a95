"""Build libteeny_hip.so: gfx950 code objects + the C-ABI host library.

    python -m teenyformers_amd.build          # or __graft_entry__.build()

Steps:
  1. each csrc/*.hip -> _build/<name>.hsaco with `hipcc --genco` for gfx950
     (in parallel);
  2. the code objects are embedded into an assembler blob (.incbin);
  3. csrc/noalloc.hip -> _build/noalloc.o with `hipcc -c -fPIC` (host code
     plus a device part that holds only the no-allocation entry point's
     static scratch array, registered with the HIP runtime when the library
     loads);
  4. csrc/capi.cpp + the blob + noalloc.o -> teenyformers_amd/libteeny_hip.so
     (g++ against the HIP runtime).

Every HIP file is compiled with packed-fp32 instruction selection disabled
(-packed-fp32-ops): the kernels' fp32 math is issued as scalar VALU ops; and
all but the GEMM with MFMA accumulators in VGPR form (see VGPR_FORM).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libteeny_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# Order matters only for readability; capi.cpp declares the same list.
KERNEL_SOURCES = [
    "transpose", "rope", "norm", "swiglu", "embed", "fa2_f32", "fa2_fwd_bf16", "fa2_bwd_bf16",
    "llama", "decode_bf16", "linear_bf16", "gemm_bf16", "gemm_f32",
]

HIPCC_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "--genco",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-ffp-contract=fast",
    "-Wno-unused-result",
]
# keep MFMA accumulators in the VGPR file: with AGPR accumulators the
# loop-carried dK/dV sums were copied between register files every
# iteration.  The GEMM keeps them in AGPRs (its accumulators are read only
# once, at the end, and a wavefront's 128 x 128 tile needs all 256).
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
NO_VGPR_FORM = {"gemm_bf16"}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l).strip()
    if err and verbose:
        print(err, file=sys.stderr)
    return r


# Per-file additions.  The forward's row maxima read MFMA results: without
# NaNs to honour, fmaxf needs no canonicalising v_max per operand.
EXTRA_FLAGS: dict[str, list[str]] = {"fa2_fwd_bf16": ["-fno-honor-nans"]}


def _hipcc(name, verbose):
    src = os.path.join(CSRC, name + ".hip")
    out = os.path.join(BUILD, name + ".hsaco")
    vf = [] if name in NO_VGPR_FORM else VGPR_FORM
    cmd = [os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, *vf, *EXTRA_FLAGS.get(name, []),
           "-I", CSRC, src, "-o", out]
    _run(cmd, verbose)
    return out


def build(verbose: bool = False, jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, len(KERNEL_SOURCES))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda n: _hipcc(n, verbose), KERNEL_SOURCES))

    blob = os.path.join(BUILD, "co_blob.S")
    with open(blob, "w") as f:
        f.write("    .section .rodata\n")
        for name, path in zip(KERNEL_SOURCES, objs):
            f.write(f"    .balign 4096\n    .global teeny_co_{name}\n    .hidden teeny_co_{name}\nteeny_co_{name}:\n")
            f.write(f'    .incbin "{path}"\n')
            f.write(f"    .global teeny_co_{name}_end\n    .hidden teeny_co_{name}_end\nteeny_co_{name}_end:\n")
        f.write('    .section .note.GNU-stack,"",@progbits\n')
    blob_o = os.path.join(BUILD, "co_blob.o")
    _run(["gcc", "-c", blob, "-o", blob_o], verbose)

    noalloc_o = os.path.join(BUILD, "noalloc.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), "-O2", "-std=c++17", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-fPIC",
          f"-I{INCLUDE}", "-c", os.path.join(CSRC, "noalloc.hip"),
          "-o", noalloc_o], verbose)

    tmp = LIB + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{ROCM}/include",
        "-Wall", "-Wextra", "-Wno-unused-parameter",
        os.path.join(CSRC, "capi.cpp"), os.path.join(CSRC, "blaslt.cpp"), blob_o, noalloc_o,
        f"-L{ROCM}/lib", "-lhipblaslt", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
        "-o", tmp,
    ]
    _run(cmd, verbose)
    os.replace(tmp, LIB)
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
