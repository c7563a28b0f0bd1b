"""Build tests/cpp/host_sanitize: the library's host sources (capi.cpp,
kernel_shims.cpp, pjrt.cpp, cblas_sgemm.cpp) and the driver host_sanitize.cpp
compiled by g++ with AddressSanitizer and UndefinedBehaviorSanitizer, linked
with the library's compiled .hip objects (device code and launchers, built by
jules_amd/build.py into _build/, not sanitized).  Host code only: no GPU code
is built with a sanitizer."""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "jules_amd", "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
BINARY = os.path.join(HERE, "host_sanitize")
HOST_SOURCES = ["capi.cpp", "kernel_shims.cpp", "pjrt.cpp", "cblas_sgemm.cpp"]
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
CXXFLAGS = ["-O1", "-g", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}",
            "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build(verbose=False):
    sys.path.insert(0, ROOT)
    from jules_amd import build as lib_build

    os.makedirs(OBJDIR, exist_ok=True)
    dev_objs = [os.path.join(OBJDIR, s + ".o") for s in lib_build.SOURCES if s.endswith(".hip")]
    missing = [o for o in dev_objs if not os.path.exists(o)]
    if missing:
        raise RuntimeError(f"library objects missing (run jules_amd/build.py first): {missing}")
    srcs = [os.path.join(CSRC, s) for s in HOST_SOURCES] + [os.path.join(HERE, "host_sanitize.cpp")]

    def compile_one(src):
        obj = os.path.join(OBJDIR, "san_" + os.path.basename(src) + ".o")
        _run(["g++", *CXXFLAGS, *SANITIZE, "-c", src, "-o", obj], verbose)
        return obj

    with cf.ThreadPoolExecutor(max_workers=5) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = BINARY + ".tmp"
    _run(["g++", *SANITIZE, *objs, *dev_objs, f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
          "-o", tmp], verbose)
    os.replace(tmp, BINARY)
    return BINARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
