"""Build the HIP library in-tree: csrc/*.hip -> starkv_serve/libstarkv_hip.so (gfx950),
then the torch operator library csrc/torch_ops.cpp -> starkv_serve/libstarkv_torch.so
(torch.ops.starkv, linked against libstarkv_hip.so).

    python star-kv-serve_amd/build.py

Each HIP source compiles in its own hipcc process (in parallel), then one link step.
"""
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "starkv_serve", "libstarkv_hip.so")
OPS_OUT = os.path.join(HERE, "starkv_serve", "libstarkv_torch.so")
CXX = os.environ.get("CXX", "g++")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         # Packed FP32 VALU ops are kept out of every code object.
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _spills(report: str) -> list:
    """Kernels of a -Rpass-analysis=kernel-resource-usage report that use scratch memory
    (register spills): [(kernel, bytes per lane)]."""
    out, name = [], None
    for line in report.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            out.append((name, int(m.group(1))))
    return out


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    # Every kernel of the library runs from registers: a kernel that spills to scratch is a
    # build error (its instantiation must be dropped or its register use reduced).
    spills = _spills(r.stderr)
    if spills:
        raise RuntimeError(f"{src}: kernels with scratch spills: {spills}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp%d" % os.getpid()
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libstarkv_hip.so", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    build_ops(verbose)
    return OUT


def build_ops(verbose: bool = True) -> str:
    """torch_ops.cpp -> libstarkv_torch.so: host C++ over torch's headers (no device code),
    linked against libstarkv_hip.so found beside it at load time."""
    import torch
    tdir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS_OUT + ".tmp%d" % os.getpid()
    cmd = [CXX, "-std=c++17", "-O2", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-I{tdir}/include", f"-I{tdir}/include/torch/csrc/api/include",
           "-I/opt/rocm/include", os.path.join(CSRC, "torch_ops.cpp"), "-o", tmp,
           f"-L{os.path.dirname(OUT)}", "-lstarkv_hip", f"-L{tdir}/lib", "-lc10", "-ltorch_cpu", "-lc10_hip",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tdir}/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch_ops.cpp failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OPS_OUT)
    if verbose:
        print(f"built {OPS_OUT}")
    return OPS_OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
