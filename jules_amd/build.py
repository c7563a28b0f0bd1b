"""Build libjules_hip.so (gfx950) in-tree with hipcc.

Every .hip source under jules_amd/csrc and capi.cpp is compiled for gfx950 only
and linked into jules_amd/libjules_hip.so.  Flags:
  -ffp-contract=off      the fp32 epilogue reproduces the reference's separate
                         multiply/add/fma sequence; fmas are written explicitly
  -packed-fp32-ops off   no v_pk_{add,mul,fma}_f32 anywhere in the library
"""
import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(ROOT, "_build")
LIB = os.path.join(HERE, "libjules_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", f"{ROCM}/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", f"-I{INCLUDE}", f"-I{CSRC}",
          "-Wall", "-Wno-unused-function"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]

SOURCES = ["gemm_f32.hip", "gemm_bf16.hip", "flash_fwd.hip", "flash_bwd.hip", "flash_bwd_dq.hip", "flash_pad.hip", "w8a16.hip", "w8a16_packed.hip", "matmul_int8.hip",
           "rowops.hip", "mlp.hip", "calib.hip", "pjrt_ops.hip", "scratch.hip", "capi.cpp", "kernel_shims.cpp",
           "pjrt.cpp"]


def _scratch_kernels(stderr):
    """Kernels whose resource-usage remark reports scratch (register spills or
    private arrays): [(name, bytes per lane)]."""
    found, name = [], None
    for line in stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            found.append((name, int(m.group(1))))
    return found


def _compile(src, verbose):
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJDIR, src + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    remarks = ["-Rpass-analysis=kernel-resource-usage"] if src.endswith(".hip") else []
    cmd = [HIPCC, *COMMON, *DEVICE, *remarks, *lang, "-c", path, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    # Several kernels issue loads from inline asm and wait for them with
    # explicit counters, so each destination register must stay untouched
    # until its wait.  A kernel that spills breaks that: the compiler may
    # store and reuse such a register while the load is in flight, and the
    # late data then overwrites whatever it holds (an address, for example).
    # No kernel of the library may use scratch.
    spills = _scratch_kernels(r.stderr)
    if spills:
        raise RuntimeError(f"{src}: kernels use scratch (register spills), which the "
                           f"asm-issued loads cannot tolerate: {spills}")
    if verbose:
        err = "\n".join(l for l in r.stderr.splitlines() if "kernel-resource-usage" not in l)
        if err.strip():
            print(err, file=sys.stderr)
    if src.endswith(".hip"):
        _check_lds_waits(src, path, lang, verbose)
    return obj


def _isa_check():
    """isa_check.py beside this file, loaded by path (this script also runs
    outside the package, and the package's own import loads the library)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("jules_isa_check", os.path.join(HERE, "isa_check.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _check_lds_waits(src, path, lang, verbose):
    """The same source as gfx950 assembly, checked by isa_check: no register
    an LDS read is still filling may be read, copied or reused before the
    wait that covers it (the asm-issued reads are invisible to the
    compiler's own waits)."""
    check_asm = _isa_check().check_asm

    asm = os.path.join(OBJDIR, src + ".s")
    cmd = [HIPCC, *COMMON, *DEVICE, *lang, "--cuda-device-only", "-S", path, "-o", asm]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src}:\n{r.stdout}\n{r.stderr}")
    with open(asm) as fh:
        bad = check_asm(fh.read())
    if bad:
        lines = [f"  {k[:70]}: line {ln}: {t}" for k, v in bad.items() for ln, t in v[:3]]
        raise RuntimeError(f"{src}: instructions touch registers an LDS read is still "
                           f"filling ({sum(len(v) for v in bad.values())} found):\n" +
                           "\n".join(lines))


def build(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    _build_cblas(verbose)
    _build_selftests(verbose)
    return LIB


CBLAS_LIB = os.path.join(HERE, "libjules_cblas.so")


def _build_cblas(verbose):
    """libjules_cblas.so: the cblas_sgemm symbol (include/jules_cblas.h), a
    host-only layer over libjules_hip.so, kept in its own library so that
    loading libjules_hip.so never interposes a BLAS."""
    tmp = CBLAS_LIB + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-fPIC", "-shared", f"-I{INCLUDE}",
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", os.path.join(CSRC, "cblas_sgemm.cpp"),
           f"-L{HERE}", "-ljules_hip", f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN",
           f"-Wl,-rpath,{ROCM}/lib", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on cblas_sgemm.cpp:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CBLAS_LIB)


def _build_selftests(verbose):
    """Host-only C++ test programs tests/cpp/<name>_selftest.cpp, linked
    against the library and the HIP runtime (g++; they allocate device
    buffers to call the library with)."""
    cdir = os.path.join(ROOT, "tests", "cpp")
    if not os.path.isdir(cdir):
        return
    for f in sorted(os.listdir(cdir)):
        if not f.endswith("_selftest.cpp"):
            continue
        src = os.path.join(cdir, f)
        out = os.path.join(cdir, f[:-4])
        cmd = ["g++", "-O2", "-std=c++17", "-Wall", f"-I{INCLUDE}", "-D__HIP_PLATFORM_AMD__",
               f"-I{ROCM}/include", src, f"-L{HERE}", "-ljules_hip", f"-L{ROCM}/lib",
               "-lamdhip64", "-Wl,-rpath,$ORIGIN/../../jules_amd", f"-Wl,-rpath,{ROCM}/lib",
               "-o", out]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"g++ failed on {src}:\n{r.stdout}\n{r.stderr}")
    # a plain C caller that binds cblas_sgemm through dlopen, as a JIT's
    # process-symbol lookup would (no link-time dependency on the library)
    src = os.path.join(cdir, "cblas_dlopen.c")
    if os.path.exists(src):
        cmd = ["gcc", "-O2", "-std=c11", "-Wall", src, "-ldl", "-lm", "-o", os.path.join(cdir, "cblas_dlopen")]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"gcc failed on {src}:\n{r.stdout}\n{r.stderr}")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
