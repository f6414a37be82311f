"""Build libbc2n.so (all HIP sources, gfx950 only) in-tree.

Each translation unit is compiled by hipcc in parallel into
bindcraft2_amd/_build/, then linked into bindcraft2_amd/libbc2n.so.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libbc2n.so")
SOURCES = ["runtime.cpp", "ln.hip", "flash.hip", "ew.hip", "triattn.hip", "trimul.hip", "transition.hip",
           "msa.hip", "opm.hip", "evoformer.hip", "ipa.hip", "msaglobal.hip", "contract.hip", "tplembed.hip",
           "embed.hip", "heads.hip", "designstep.hip", "seqfeat.hip", "confidence.hip",
           "probe.hip", "capi.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no packed-FP32 VALU forms on this target (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
# Per-file extras.  The attention kernels run VALU work (softmax, masking) on
# every MFMA result: MFMA writing VGPRs directly saves the AGPR->VGPR moves.
EXTRA = {
    "flash.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, "-x", "hip", *FLAGS, *EXTRA.get(src, []), "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, len(SOURCES))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
