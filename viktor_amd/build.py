"""Build libviktor_hip.so (all kernels of viktor_amd/csrc) for gfx950 with hipcc.

Usage: python -m viktor_amd.build [--jobs N] [--phase-stamps]

The library is written next to this file, in-tree, so it travels with the repository snapshot.
--phase-stamps also links libviktor_hip_stamps.so, a profiling build whose decode-step product kernels
(csrc/skinny_gemm.hip, compiled with -DVK_PHASE_STAMPS) write per-workgroup phase timestamps; everything else
in it is the product build's objects.
Every source is compiled to an object in parallel, then linked once. The HIP runtime is resolved by
soname (libamdhip64.so.7) at load time, so after `import torch` the library binds to the runtime
torch already loaded and shares its streams and graphs.
"""

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB = os.path.join(HERE, "libviktor_hip.so")
STAMPS_LIB = os.path.join(HERE, "libviktor_hip_stamps.so")
STAMPED_SOURCE = "skinny_gemm.hip"
OBJ_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU ops stay off: the compiler is not to emit v_pk_{add,mul,fma}_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unknown-pragmas",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is needed to build the HIP kernels)")
    return path


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src, defines=()):
    tag = "_stamps" if defines else ""
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + tag + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *[f"-D{d}" for d in defines], f"-I{INCLUDE}", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the gfx feature flag above; that warning is expected
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def _link(objs, out):
    tmp = out + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)


def build(jobs=None, verbose=False, phase_stamps=False):
    """Compile every kernel source and link libviktor_hip.so (and, with phase_stamps, the profiling build
    libviktor_hip_stamps.so); returns the product library's path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    tasks = [(s, ()) for s in srcs]
    if phase_stamps:
        tasks.append((os.path.join(CSRC, STAMPED_SOURCE), ("VK_PHASE_STAMPS",)))
    with ThreadPoolExecutor(max_workers=jobs or min(8, len(tasks))) as ex:
        results = list(ex.map(lambda t: _compile(*t), tasks))
    if verbose:
        for obj, err in results:
            if err.strip():
                print(err, file=sys.stderr)
    objs = [o for o, _ in results[:len(srcs)]]
    _link(objs, LIB)
    if phase_stamps:
        stamped = results[-1][0]
        _link([stamped if os.path.basename(s) == STAMPED_SOURCE else o for s, o in zip(srcs, objs)], STAMPS_LIB)
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--phase-stamps", action="store_true", help="also link the phase-timestamp profiling build")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.phase_stamps))


if __name__ == "__main__":
    main()
