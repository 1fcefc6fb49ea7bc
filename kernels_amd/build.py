"""Build libkq.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Every source under kernels_amd/csrc is compiled for gfx950 only, with packed
FP32 instructions disabled (-Xclang -target-feature -Xclang -packed-fp32-ops),
and linked into kernels_amd/_lib/libkq.so. Runs on a CPU-only machine
(hipcc cross-compiles the device code).
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIB_DIR, "libkq.so")
DRV_SRC = os.path.join(HERE, "drivers")
BIN_DIR = os.path.join(HERE, "_bin")
DRIVERS = ("int4gemv", "vqgemv", "moefused", "moepipe")
ARCH = "gfx950"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wextra", "-Wshadow", "-Werror=shadow", "-Werror=unused-parameter",
         "-Wno-unused-function", "-Wno-sign-compare",
         "-I", os.path.join(ROOT, "include"), "-I", CSRC]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))


def _compile(src, verbose):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
    cmd = [HIPCC] + FLAGS + lang + ["-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines()
                     if "packed-fp32-ops" not in l and l.strip())
    return obj, warn


def _driver(name, verbose):
    """The C++ host drivers: host-only code over the C ABI, linked against
    libkq.so (found through an $ORIGIN-relative rpath) and the HIP runtime."""
    out = os.path.join(BIN_DIR, name)
    cmd = [os.path.join(ROCM, "llvm", "bin", "clang++"), "-O2", "-std=c++20", "-Wall", "-Wextra",
           "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROCM, "include"), os.path.join(DRV_SRC, name + ".cpp"),
           "-o", out + ".tmp", "-L", LIB_DIR, "-lkq", "-L", os.path.join(ROCM, "lib"),
           "-lamdhip64", "-pthread", "-Wl,-rpath,$ORIGIN/../_lib",
           "-Wl,-rpath," + os.path.join(ROCM, "lib")]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"driver build failed for {name}:\n{r.stdout}\n{r.stderr}")
    if verbose and r.stderr.strip():
        print(r.stderr, flush=True)
    os.replace(out + ".tmp", out)
    return out


def build_drivers(verbose: bool = False):
    os.makedirs(BIN_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(DRIVERS)) as ex:
        return list(ex.map(lambda n: _driver(n, verbose), DRIVERS))


def _fresh(src):
    """True if src's object is newer than src and every header it may include."""
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    if not os.path.exists(obj):
        return False
    deps = [src] + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    deps.append(os.path.join(ROOT, "include", "kq.h"))
    return all(os.path.getmtime(obj) > os.path.getmtime(d) for d in deps)


def build(verbose: bool = False, jobs: int = 0, incremental: bool = False) -> str:
    """Compile every source (incremental=True: only those whose object is
    older than the source or a header) and link libkq.so and the drivers."""
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    todo = [s for s in srcs if not (incremental and _fresh(s))]
    jobs = jobs or min(max(1, len(todo)), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for _, warn in ex.map(lambda s: _compile(s, verbose), todo):
            if warn and verbose:
                print(warn, flush=True)
    objs = [os.path.join(OBJ, os.path.basename(s) + ".o") for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    build_drivers(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, incremental="-i" in sys.argv))
