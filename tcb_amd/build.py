"""Build libtrhip.so (HIP, gfx950) and the CPU oracle in-tree.

Used by __graft_entry__.build(); runnable directly: python -m tcb_amd.build
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtrhip.so")

SOURCES = ["api.hip", "wstore.hip", "gemv.hip", "gemv_fast.hip", "gemm_rows.hip", "actq.hip", "actq_mfma.hip",
           "swiglu.hip", "probe.hip", "prefill.hip", "rows16.hip", "actq6.hip", "actq4.hip",
           "io16.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: no multiply-add is fused unless written as fmaf (bit-exact rounding order).
# -packed-fp32-ops off: no v_pk_*_f32 instructions are generated.
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("command failed: %s\n%s%s" % (" ".join(cmd), r.stdout, r.stderr))
    return r


def build_lib(jobs=None):
    os.makedirs(OBJ, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        _run([HIPCC] + FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=jobs or min(8, len(SOURCES))) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
    return os.path.join(ROOT, "oracle", "liboracle.so")


def main():
    print(build_oracle())
    print(build_lib())


if __name__ == "__main__":
    sys.exit(main())
