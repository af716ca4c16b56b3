"""Build libmeshy_amd.so in-tree with hipcc for gfx950.

    python -m meshy_amd.build

Each source compiles to its own object under meshy_amd/_build/ (in parallel),
then one link produces meshy_amd/libmeshy_amd.so next to this file.  The
CPython extensions meshy_amd._pyio (host code over Python objects) and
meshy_amd._stage (host code over libtorch's tensor type), no device code in
either, are built beside it with the host compiler.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "libmeshy_amd.so")

SOURCES = ("capi.cpp", "plan.cpp", "hostio.cpp", "logprob.hip", "topk.hip", "distill.hip", "pack.hip", "ppo.hip", "gae.hip", "critic.hip", "ragged.hip", "synth.hip", "order.hip")

PYIO_SRC = "pyio.cpp"
PYIO_OUT = os.path.join(HERE, "_pyio" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
STAGE_SRC = "stage.cpp"
STAGE_OUT = os.path.join(HERE, "_stage" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
AUTOGRAD_SRC = "autograd.cpp"
AUTOGRAD_OUT = os.path.join(HERE, "_autograd" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

ARCH = os.environ.get("MESHY_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU forms are kept out of the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build libmeshy_amd)")
    return path


# Per-source flags.  The synthetic-logit generator must give the same bits on
# the host and the device, so no multiply and add may be fused implicitly.
EXTRA_FLAGS = {"synth.hip": ["-ffp-contract=off"]}


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    # .hip sources are compiled for the device and the host; the .cpp sources
    # are host code only (no device pass).
    lang = ["-x", "hip"] if src.endswith(".hip") else ["--offload-host-only"]
    cmd = [hipcc(), *COMMON_FLAGS, *EXTRA_FLAGS.get(src, []), *lang, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the device-only feature flag.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build_pyio(verbose: bool = False) -> str:
    """Compile the CPython extension meshy_amd._pyio; returns its path."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler found for meshy_amd._pyio")
    tmp = PYIO_OUT + ".tmp"
    cmd = [cxx, "-O3", "-std=c++17", "-shared", "-fPIC", "-pthread", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           os.path.join(CSRC, PYIO_SRC), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cxx} failed on {PYIO_SRC}:\n{res.stderr}")
    os.replace(tmp, PYIO_OUT)
    return PYIO_OUT


def build_stage(verbose: bool = False) -> str:
    """Compile the CPython extension meshy_amd._stage (host code over libtorch's
    tensor type: reads each sample tensor's pointer, dtype and shape without a
    Python attribute call); returns its path."""
    import torch
    from torch.utils import cpp_extension

    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler found for meshy_amd._stage")
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(bool(getattr(torch._C, "_GLIBCXX_USE_CXX11_ABI", True)))
    tmp = STAGE_OUT + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in cpp_extension.include_paths()], f"-I{sysconfig.get_paths()['include']}",
           os.path.join(CSRC, STAGE_SRC), "-o", tmp, f"-L{libdir}", "-ltorch_python", "-ltorch_cpu", "-lc10",
           f"-Wl,-rpath,{libdir}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cxx} failed on {STAGE_SRC}:\n{res.stderr[-4000:]}")
    os.replace(tmp, STAGE_OUT)
    return STAGE_OUT


def _torch_host_flags() -> tuple[list[str], str]:
    """g++ flags for host code over libtorch's headers, and torch's lib folder."""
    import torch
    from torch.utils import cpp_extension

    abi = int(bool(getattr(torch._C, "_GLIBCXX_USE_CXX11_ABI", True)))
    flags = [f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *[f"-I{p}" for p in cpp_extension.include_paths()],
             f"-I{sysconfig.get_paths()['include']}"]
    return flags, os.path.join(os.path.dirname(torch.__file__), "lib")


def _rocm_include() -> str:
    """The ROCm include folder (beside hipcc's bin folder)."""
    return os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(hipcc()))), "include")


def compile_autograd(verbose: bool = False) -> str:
    """Compile csrc/autograd.cpp (the C++ autograd nodes of the loss drop-ins)
    to an object file; returns its path."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler found for meshy_amd._autograd")
    flags, _ = _torch_host_flags()
    obj = os.path.join(BUILD_DIR, "autograd.o")
    # c10's HIP stream header reads the HIP runtime's declarations.
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-Wall", "-c", "-D__HIP_PLATFORM_AMD__", *flags,
           f"-I{_rocm_include()}", f"-I{os.path.join(ROOT, 'include')}", os.path.join(CSRC, AUTOGRAD_SRC), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cxx} failed on {AUTOGRAD_SRC}:\n{res.stderr[-4000:]}")
    return obj


def link_autograd(obj: str, verbose: bool = False) -> str:
    """Link meshy_amd._autograd against libmeshy_amd.so (found beside it at run
    time) and libtorch; returns its path."""
    cxx = shutil.which("g++") or shutil.which("c++")
    _, libdir = _torch_host_flags()
    tmp = AUTOGRAD_OUT + ".tmp"
    cmd = [cxx, "-shared", obj, "-o", tmp, f"-L{HERE}", "-lmeshy_amd", f"-L{libdir}", "-ltorch_python",
           "-ltorch_cpu", "-lc10_hip", "-lc10", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of meshy_amd._autograd failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, AUTOGRAD_OUT)
    return AUTOGRAD_OUT


def build(verbose: bool = False) -> str:
    """Compile every source and link libmeshy_amd.so (and build meshy_amd._pyio);
    returns the library's path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES) + 3, os.cpu_count() or 1)) as ex:
        stage = ex.submit(build_stage, verbose)
        pyio = ex.submit(build_pyio, verbose)
        autograd = ex.submit(compile_autograd, verbose)
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
        pyio.result()
        stage.result()
        autograd_obj = autograd.result()
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    link_autograd(autograd_obj, verbose)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
