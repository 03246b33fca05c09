"""Build the gfx950 HIP library libblt_hip.so in-tree with hipcc.

Every .hip file under csrc/ is compiled for gfx950 (device code plus host
launchers and the C ABI) and linked into blt-burn_amd/libblt_hip.so.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libblt_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # code object v5: loadable by the ROCm 7.0 HIP runtime that torch bundles
    # as well as by ROCm 7.2's
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast", "-Wall", "-Wno-unused-function",
    "-I", os.path.join(HERE, "..", "include"),
]
# per-file additions
FILE_FLAGS = {
    # keep MFMA sources and results in arch VGPRs: the attention softmax works
    # on the score accumulators with VALU ops, and results parked in AGPRs cost
    # a v_accvgpr read/write per value per tile (the GEMMs keep their
    # accumulators in AGPRs where the 4-wave tiles need the room)
    "k_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(OBJ, f[:-4] + ".o") for f in srcs]
    jobs = [[HIPCC] + FLAGS + FILE_FLAGS.get(s, []) + ["-c", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(srcs, objs)]
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
