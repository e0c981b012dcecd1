"""Build libloki_moe.so (HIP, gfx950) in-tree with hipcc.

Flags that matter for parity: -ffp-contract=off (the fp32/fp64 rounding sequences are a contract shared with the CPU
checker; HIP's default would fuse a*b+c into FMAs) and no fast-math. Packed FP32 VALU ops are disabled
(-packed-fp32-ops): every fp32 op stays a scalar-lane op.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIBDIR, "libloki_moe.so")
SOURCES = ["quant.hip", "router.hip", "dispatch.hip", "iq2_gemv.hip", "moe_decode.hip", "moe_decode1.hip", "moe_prefill.hip", "pack.hip", "kquant.hip", "kq_gemm.hip", "gguf.hip", "fused_layer.hip", "compat.hip"]
HEADERS = ["moe_common.h", "moe_device.h", "moe_kernels.h", "fl_ctx.h", "iq2xxs_grid.inc"]
ARCH = os.environ.get("LOKI_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-parameter",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libloki_moe)")


def build(verbose=False, jobs=None):
    """Compile every source to an object (in parallel), then link the shared library. Always rebuilds."""
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    cc = hipcc()
    inc = ["-I" + CSRC, "-I" + os.path.join(os.path.dirname(HERE), "include")]
    procs = []
    objs = []
    for s in SOURCES:
        src = os.path.join(CSRC, s)
        obj = os.path.join(objdir, s.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [cc] + HIPCC_FLAGS + inc + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((s, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for s, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
        if p.returncode != 0:
            failed.append((s, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        for s, t in failed:
            sys.stderr.write("---- %s\n%s\n" % (s, t))
        raise RuntimeError("hipcc failed for: " + ", ".join(s for s, _ in failed))
    tmp = LIB + ".tmp"
    cmd = [cc, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
