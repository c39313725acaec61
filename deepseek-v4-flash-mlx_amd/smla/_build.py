"""Builds libsmla.so in-tree with hipcc for gfx950 (one object per source, compiled in parallel,
then linked)."""
import os
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(_HERE), "csrc")
SOURCES = ["attn.hip", "attn_decode.hip", "indexer.hip", "topk.hip", "pool.hip", "qat.hip", "linear.hip",
           "gemm.hip", "capi.hip"]
OUT = os.path.join(_HERE, "libsmla.so")
# linker version script: only the smla_* C entry points are exported
EXPORTS = os.path.join(CSRC, "libsmla.map")

FLAGS = ["-O3", "--offload-arch=gfx950", "-std=c++17", "-fPIC",
         # packed fp32 VALU ops are disabled for every kernel (hipcc's host pass warns that it does
         # not know the feature; that is harmless)
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

# per-source additions.  attn_decode.hip: MFMA accumulators in VGPRs (its online-softmax rescale
# touches them with VALU ops; with AGPR accumulators every P.V step would copy them both ways)
EXTRA = {"attn_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def _compile(hipcc, src, obj):
    cmd = [hipcc, *FLAGS, *EXTRA.get(os.path.basename(src), []), "-c", "-o", obj, src]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    return " ".join(cmd)


def build(verbose=False):
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    missing = [s for s in srcs if not os.path.exists(s)]
    if missing:
        raise FileNotFoundError("libsmla sources missing: " + ", ".join(missing))
    with tempfile.TemporaryDirectory(prefix="smla_build_") as tmpd:
        objs = [os.path.join(tmpd, os.path.basename(s) + ".o") for s in srcs]
        with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            cmds = list(ex.map(lambda so: _compile(hipcc, *so), zip(srcs, objs)))
        tmp = OUT + ".tmp"
        link = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", f"-Wl,--version-script={EXPORTS}", "-o", tmp,
                *objs]
        res = subprocess.run(link, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    if verbose:
        for c in cmds:
            print(c)
        print(" ".join(link))
    os.replace(tmp, OUT)
    return OUT
