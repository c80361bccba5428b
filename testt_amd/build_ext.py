"""Builds libsoupk.so (the gfx950 kernels behind the C ABI in include/soupk.h) in place.

    python -m testt_amd.build_ext          # or __graft_entry__.build()

hipcc cross-compiles for gfx950 without a GPU.  Every source in testt_amd/csrc/*.hip becomes
one object under testt_amd/_build/, and the objects are linked into testt_amd/libsoupk.so,
the file the Python layer loads (it travels with the source tree; it is not installed).
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB_NAME = "libsoupk.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"

# -ffp-contract=off: products and sums are rounded one at a time (the NF4 closed form is
#   bit-exact only that way, and the other kernels then round like the eager PyTorch path).
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 generated.
# -amdgpu-mfma-vgpr-form: MFMA accumulators in ordinary VGPRs.  Without it the compiler put the
#   MFMA results of the attention, LoRA and NF4-GEMM kernels in AGPRs and copied them to and
#   from VGPRs around every use (v_accvgpr_read/write: 192 in the attention forward, 424 in
#   the backward), although their register budgets fit in VGPRs alone.  Measured on MI355X:
#   attention backward 45.9 -> 44.8 us, the rest unchanged within noise; results identical.
COMPILE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall", "-Werror=return-type",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is expected under /opt/rocm)")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(hipcc, src, build_dir, defines):
    obj = os.path.join(build_dir, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc, *COMPILE_FLAGS, *[f"-D{d}" for d in defines], "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return obj


def build(verbose=False, defines=(), out=None):
    """Compile every kernel source and link libsoupk.so; returns the library path.

    `defines` (e.g. "SOUPK_HEAD_PREFETCH=8") override the launch-shape constants of the
    sources; with `out`, the library is written there instead (a tuning variant), from its
    own object directory."""
    hipcc = _hipcc()
    lib_path = out or LIB_PATH
    build_dir = BUILD if out is None else os.path.splitext(out)[0] + "_build"
    os.makedirs(build_dir, exist_ok=True)
    srcs = sources()
    jobs = max(1, min(len(srcs), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(lambda s: _compile(hipcc, s, build_dir, defines), srcs))
    tmp = lib_path + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           "-lhipblaslt"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {LIB_NAME} failed:\n{proc.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path} from {len(srcs)} sources", flush=True)
    return lib_path


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
