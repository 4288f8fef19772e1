"""Build the gfx950 hot-tier library libhotcold_hip.so in-tree.

    python hotcold-kv-cache_amd/build_native.py [--jobs N]

Compiles every csrc/*.hip for gfx950 with hipcc and every csrc/*.cpp (host
code: the cold store) with g++, one object per file, in parallel, and links
hotcold_kv/_lib/libhotcold_hip.so.  No torch involvement: the library's ABI
is plain C (include/hotcold_hip.h).
"""

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT_DIR = os.path.join(HERE, "hotcold_kv", "_lib")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libhotcold_hip.so"

ARCH = os.environ.get("HOTCOLD_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 VALU forms (v_pk_fma_f32 & co.) are kept out of the code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-file extra flags.  The window-scoring kernels keep their fp64 MFMA
# accumulators in VGPRs: with the default AGPR form the compiler copies all 32
# accumulator registers between the two files on every loop iteration.
FILE_FLAGS = {
    "hc_snapkv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the hot-tier library needs ROCm's hipcc")
    return exe


# Host C++ (no device code).  AVX2 for the cold-store scans; floating-point
# contraction off so the fp64 search arithmetic is the written sequence.
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-pthread", "-mavx2", "-mf16c", "-ffp-contract=off", "-Wall", f"-I{INCLUDE}",
             f"-I{CSRC}"]


def _compile(src, obj):
    if src.endswith(".cpp"):
        cmd = [shutil.which("g++") or "g++", *CXX_FLAGS, "-c", src, "-o", obj]
    else:
        cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and "--hip-link" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed for {os.path.basename(src)}:\n{errs}")
    return errs


def build(jobs=None, verbose=True):
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip") or f.endswith(".cpp"))
    objs = [os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o") for s in srcs]
    jobs = jobs or min(8, os.cpu_count() or 4, len(srcs))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = {ex.submit(_compile, os.path.join(CSRC, s), o): s for s, o in zip(srcs, objs)}
        for f in cf.as_completed(futs):
            warn = f.result()
            if verbose and warn.strip():
                print(f"[build] {futs[f]}:\n{warn}", file=sys.stderr)
    out = os.path.join(OUT_DIR, LIB_NAME)
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objs, "-o", tmp,
           "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"[build] {out}")
    return out


BIND_SRC = os.path.join(CSRC, "bind", "hc_step_bind.cpp")
BIND_NAME = "hc_step_bind"


def build_bind(verbose=True):
    """The Python extension module of the decode loop's per-step call
    (csrc/bind/hc_step_bind.cpp: host C++ against torch's headers, linked to
    libhotcold_hip.so beside it), built into OUT_DIR next to the library.
    Build the library first."""
    import torch.utils.cpp_extension as ce

    lib = os.path.join(OUT_DIR, LIB_NAME)
    if not os.path.exists(lib):
        raise RuntimeError(f"build the library ({lib}) before its binding")
    bdir = os.path.join(OBJ_DIR, "bind")
    os.makedirs(bdir, exist_ok=True)
    # runpath: the library beside the installed module ($ORIGIN), and from
    # the build directory (where load() imports it once) the same library;
    # '$$' is ninja's escape of '$' and '\' the shell's
    rel = os.path.relpath(OUT_DIR, bdir)
    ce.load(name=BIND_NAME, sources=[BIND_SRC], build_directory=bdir, extra_cflags=["-O3", f"-I{INCLUDE}"],
            extra_ldflags=[f"-L{OUT_DIR}", "-lhotcold_hip", f"-Wl,-rpath,\\$$ORIGIN:\\$$ORIGIN/{rel}"],
            verbose=False)
    out = os.path.join(OUT_DIR, BIND_NAME + ".so")
    shutil.copyfile(os.path.join(bdir, BIND_NAME + ".so"), out + ".tmp")
    os.replace(out + ".tmp", out)
    if verbose:
        print(f"[build] {out}")
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs)
    build_bind()
