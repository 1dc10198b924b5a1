"""Builds libtg_fp8.so (the C ABI of include/tg_fp8.h) for gfx950 with hipcc.

Usage: ``python train-gpt_amd/build.py`` (or ``__graft_entry__.build()``).
Each ``csrc/*.hip`` compiles to an object in ``csrc/_build`` in parallel; the
objects link into ``train-gpt_amd/libtg_fp8.so``.  hipcc cross-compiles for
gfx950 without a GPU.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJDIR = os.path.join(CSRC, "_build")
LIB = os.path.join(HERE, "libtg_fp8.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["quant.hip", "rmsnorm.hip", "gemm_fp8.hip", "gemm_bf16.hip", "attention.hip",
           "xent.hip", "block_generic.hip", "noalloc.hip"]

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 (plain f32 VALU only).
# -ffp-contract=off: every multiply/add in the numeric contract stays a single
#   IEEE operation unless written as an explicit fma.
# correctly rounded f32 divide/sqrt: the quantizer's x / s is an IEEE divide.
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source flags.  gemm_fp8.hip: MFMA results in VGPRs even where one wave
# per SIMD would let the compiler use AGPRs (its short-K kernel promotes every
# MFMA result with VALU FMAs, which read VGPRs only).
EXTRA_FLAGS = {"gemm_fp8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build_library(verbose: bool = False) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    _check_stubs(tmp)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def _check_stubs(lib: str) -> None:
    """Fail on a kernel whose host launch stub the compiler did not emit: hipcc
    then links a library with an undefined __device_stub__ symbol that only
    fails when the library is loaded."""
    r = subprocess.run(["nm", "-u", lib], capture_output=True, text=True)
    missing = [ln.split()[-1] for ln in r.stdout.splitlines() if "__device_stub__" in ln]
    if missing:
        raise RuntimeError(f"{lib}: {len(missing)} kernel stubs undefined, e.g. {missing[0]}")


PROBE_SRCS = [os.path.join(CSRC, "probe", f) for f in ("io_floor.hip", "gemv_stream.hip", "quant_floor.hip")]
PROBE_LIB = os.path.join(HERE, "libtg_probe.so")


def build_probe(verbose: bool = False) -> str:
    """Compile bench.py's floor probes (csrc/probe/io_floor.hip: the fused norm's
    I/O; csrc/probe/gemv_stream.hip: the direct decode GEMV's loads) into
    libtg_probe.so, linked against libtg_fp8.so for its error reporting.  It is
    measurement tooling: nothing in the package loads it."""
    tmp = PROBE_LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, "-shared", *PROBE_SRCS, "-L", HERE, "-ltg_fp8", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {PROBE_LIB}")
    return PROBE_LIB


FFI_SRC = os.path.join(CSRC, "ffi", "tg_xla_ffi.cc")
FFI_CORE = os.path.join(CSRC, "ffi", "tg_ffi_core.h")
FFI_CORE_SHIM = os.path.join(CSRC, "ffi", "tg_ffi_core_shim.cc")
FFI_LIB = os.path.join(HERE, "libtg_xla_ffi.so")
FFI_CORE_LIB = os.path.join(HERE, "libtg_ffi_core.so")
CXX = os.environ.get("CXX", "g++")


def build_ffi_core(verbose: bool = False) -> str:
    """Compile the XLA FFI handlers' logic (csrc/ffi/tg_ffi_core.h) with its C-ABI
    shim into libtg_ffi_core.so, linked against libtg_fp8.so.  Host code only
    (the C ABI takes streams as void*), so the host compiler builds it; it needs
    no jaxlib.  Test tooling: the tests run the handlers' checks, dispatch and
    workspace handling through it; nothing in the package loads it."""
    root = os.path.dirname(HERE)
    tmp = FFI_CORE_LIB + ".tmp"
    cmd = [CXX, "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-I", os.path.join(root, "include"),
           FFI_CORE_SHIM, "-L", HERE, "-ltg_fp8", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"FFI core shim failed to build:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, FFI_CORE_LIB)
    if verbose:
        print(f"built {FFI_CORE_LIB}")
    return FFI_CORE_LIB


def build_xla_ffi(verbose: bool = False):
    """Compile the XLA FFI handlers (csrc/ffi/tg_xla_ffi.cc) into libtg_xla_ffi.so.

    They need xla/ffi/api/ffi.h, which jaxlib ships (jax.ffi.include_dir()).
    Where jax is not importable the step is skipped with a message and None is
    returned; the C ABI (libtg_fp8.so) does not depend on it.
    """
    try:
        import jax
        inc = jax.ffi.include_dir()
    except Exception as e:  # jax / jaxlib absent, or too old for jax.ffi
        print(f"skipping the XLA FFI handlers: jax.ffi.include_dir() is unavailable "
              f"({e.__class__.__name__}: {e})")
        return None
    root = os.path.dirname(HERE)
    cmd = [HIPCC, "-std=c++17", "-O2", "-fPIC", "-shared", "-I", inc, "-I", os.path.join(root, "include"),
           FFI_SRC, "-L", HERE, "-ltg_fp8", "-Wl,-rpath,$ORIGIN", "-o", FFI_LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"XLA FFI handlers failed to build:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {FFI_LIB}")
    return FFI_LIB


if __name__ == "__main__":
    build_library(verbose=True)
    build_probe(verbose=True)
    build_ffi_core(verbose=True)
    build_xla_ffi(verbose=True)
    sys.exit(0)
