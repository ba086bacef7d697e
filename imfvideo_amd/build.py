"""Build the gfx950 C-ABI library ``libsla2hip.so`` in-tree with hipcc.

Run as ``python -m imfvideo_amd.build``.  Each ``csrc/*.hip`` file compiles to
an object under ``imfvideo_amd/_build/`` and the objects link into
``imfvideo_amd/libsla2hip.so``.  ``quant_route.hip`` is compiled with
``-ffp-contract=off``: its fp32 sums and dot products must round in the
written order to stay bit-identical with the CPU restatement.
"""

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsla2hip.so")
ARCH = os.environ.get("SLA2H_ARCH", "gfx950")

SOURCES = {
    "quant_route.hip": ["-ffp-contract=off"],
    "states.hip": [],
    # accumulators in VGPR-form MFMA: no AGPR round trips across the key loop.
    # The key loops branch to a rare rescale of the accumulators on a
    # wave-uniform condition; left unstructured, those branches cost no
    # extra live ranges (256 -> 238 VGPRs and no scratch in fwd_jvp).
    "attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1",
                 "-mllvm", "-structurizecfg-skip-uniform-regions=true"],
    "attn_train.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1",
                       "-mllvm", "-structurizecfg-skip-uniform-regions=true"],
    "attn_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "mla_glue.hip": [],
    "block_train.hip": [],
}

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # packed fp32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _run(cmd):
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose=False):
    """Compile every HIP source for gfx950 and link libsla2hip.so; returns its path."""
    cc = hipcc()
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    for src, extra in SOURCES.items():
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        cmd = [cc, *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        out = _run(cmd)
        if verbose and out.strip():
            print(out)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
