"""Build the HIP library ``torch_pesq/_lib/libpesq_hip.so`` for gfx950.

Every ``csrc/*.hip`` translation unit is compiled by ``hipcc`` into an object
and linked into one shared library with a plain C ABI (``include/pesq_hip.h``).
``csrc/torch_autograd.cpp``, the PyTorch autograd node of the fused pipeline,
is compiled by the host compiler against PyTorch's headers into the extension
module ``torch_pesq/_lib/_pesq_torch.so``, which links the library.  Both are
built in-tree so that they travel with the source tree.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "torch_pesq" / "_lib"
LIB = OUT_DIR / "libpesq_hip.so"
EXT = OUT_DIR / "_pesq_torch.so"
EXT_SRC = CSRC / "torch_autograd.cpp"
OBJ_DIR = HERE / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = os.environ.get("PESQ_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # packed fp32 instructions are disabled for all device code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: Path, verbose: bool) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed on {src.name}")
    # the host pass does not know the packed-fp32 feature; keep its warning quiet
    noise = "packed-fp32-ops"
    for line in (proc.stdout + proc.stderr).splitlines():
        if line.strip() and noise not in line:
            print(line)
    return obj


def _torch_flags():
    """Compile and link flags of a PyTorch (ROCm) C++ extension module."""

    import sysconfig

    import torch
    from torch.utils.cpp_extension import include_paths

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    cflags = [
        "-O2",
        "-std=c++17",
        "-fPIC",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-DTORCH_EXTENSION_NAME=_pesq_torch",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        *[f"-I{p}" for p in include_paths()],
        f"-I{sysconfig.get_paths()['include']}",
        "-I/opt/rocm/include",
        f"-I{ROOT / 'include'}",
    ]
    ldflags = [
        "-shared",
        f"-L{torch_lib}",
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-ltorch_python",
        "-lamdhip64",  # the HIP runtime PyTorch loads (graph capture and replay)
        f"-L{OUT_DIR}",
        "-lpesq_hip",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    return cflags, ldflags


def _run(cmd, verbose: bool, what: str):
    if verbose:
        print(" ".join(map(str, cmd)), flush=True)
    proc = subprocess.run(list(map(str, cmd)), capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"{what} failed")


def build(verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    cflags, ldflags = _torch_flags()
    ext_obj = OBJ_DIR / (EXT_SRC.stem + ".o")

    def compile_ext():
        _run([CXX, *cflags, "-c", EXT_SRC, "-o", ext_obj], verbose, f"{CXX} on {EXT_SRC.name}")
        return ext_obj

    workers = min(len(sources) + 1, os.cpu_count() or 1, 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        ext_job = pool.submit(compile_ext)
        objects = list(pool.map(lambda s: _compile(s, verbose), sources))
        ext_job.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run(
        [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libpesq_hip.so",
         *objects, "-o", tmp],
        verbose,
        "linking libpesq_hip.so",
    )
    os.replace(tmp, LIB)
    tmp = EXT.with_suffix(".so.tmp")
    _run([CXX, ext_obj, *ldflags, "-o", tmp], verbose, "linking _pesq_torch.so")
    os.replace(tmp, EXT)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
