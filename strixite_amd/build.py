"""Builds libstrixite_amd.so (every HIP source under csrc/, gfx950) in-tree, plus the CPU checker under oracle/.

    python -m strixite_amd.build          # or __graft_entry__.build()

hipcc cross-compiles for gfx950 without a GPU. Objects go to strixite_amd/_build/ (git-ignored); the shared library
lands next to this file, where strixite_amd/__init__.py loads it from.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libstrixite_amd.so")
ARCH = os.environ.get("SX_OFFLOAD_ARCH", "gfx950")

# Packed FP32 (v_pk_*_f32) is kept off in every HIP compile: some of its forms have given wrong results on these
# boxes. The host pass warns that it does not know the feature; that is harmless.
HIPFLAGS = [
    "-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)):
            return c
    return "hipcc"


def _compile(src):
    obj = os.path.join(OUT, os.path.basename(src) + ".o")
    cmd = [hipcc(), *HIPFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj


def build(jobs=None, verbose=True):
    os.makedirs(OUT, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1), 16)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    if verbose:
        print(f"built {LIB} from {len(srcs)} HIP sources for {ARCH}")
    return LIB


def build_oracle():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


if __name__ == "__main__":
    build()
    build_oracle()
    sys.exit(0)
