"""Build recipe of the native library ``libflashcodec_amd.so`` (gfx950).

Every ``csrc/*.hip`` file is compiled by hipcc to an object in
``flashcodec_amd/_build/`` (in parallel) and linked in-tree, next to this
file, so the library travels with the source tree.  Flags:

* ``--offload-arch=gfx950``: MI355X only, no other targets.
* ``-ffp-contract=off``: the codec kernels rely on exactly the fused
  multiply-adds they spell out (bit-exact archive codes).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32
  instructions are generated.
* ``-mcode-object-version=5``: loadable by the ROCm runtime bundled with
  PyTorch as well as the system one.
* ``-mllvm -amdgpu-mfma-vgpr-form`` (matrix-core sources only): matrix-core
  results in ordinary VGPRs, so the softmax rescale of the accumulators needs
  no copies through the accumulation registers.
"""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libflashcodec_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build "
                           "flashcodec_amd")
    return path


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


# extra flags by source-name prefix (the matrix-core kernels' translation units)
FILE_FLAGS = {
    "fc_attn_mfma": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "fc_prefill": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def file_flags(name):
    return next((flags for prefix, flags in FILE_FLAGS.items() if name.startswith(prefix)), [])


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    extra = file_flags(os.path.basename(src))
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose=False):
    """Compile and link the library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
