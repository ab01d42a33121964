"""Build the HIP library libzerollm_hip.so in-tree for gfx950 with hipcc.

    python -m zerollm_amd.build        (also called by __graft_entry__.build())
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = ["zl_attn.hip", "zl_delta.hip", "zl_gemv_q4k.hip", "zl_gemv_q6k.hip", "zl_gemv_q8.hip", "zl_gemv_q40.hip", "zl_gemv_q50.hip", "zl_gemv_q5k.hip",
           "zl_gemv_mfma.hip", "zl_gemm_q4k.hip", "zl_gemm_q5k.hip", "zl_gemm_q6k.hip", "zl_gemm_q8.hip", "zl_gemv_rg.hip", "zl_gemv.hip", "zl_kernels.hip", "zl_sample.hip", "zl_runtime.cpp", "gguf.cpp"]
LIB = os.path.join(HERE, "libzerollm_hip.so")

# -ffp-contract=off: every f64/f32 step rounds where the reference's arithmetic rounds; fusions are explicit fma().
# -packed-fp32-ops off: no v_pk_*_f32 is generated.
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-I" + os.path.join(ROOT, "include"),
]


def build(verbose: bool = False) -> str:
    """Compile every source to an object (in parallel), then link the shared library."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    procs, objs = [], []
    for s in SOURCES:
        obj = os.path.join(objdir, os.path.splitext(s)[0] + ".o")
        objs.append(obj)
        cmd = [hipcc, *FLAGS, "-c", "-x", "hip", os.path.join(HERE, "csrc", s), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
    failed = False
    for p in procs:
        out = p.communicate()[0]
        if p.returncode != 0:
            sys.stderr.write(out)
            failed = True
    if failed:
        raise RuntimeError("hipcc failed building libzerollm_hip.so")
    tmp = LIB + ".tmp"
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp, "-lpthread"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("linking libzerollm_hip.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
