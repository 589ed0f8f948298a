"""Builds libflint_amd.so (all HIP kernels + the C ABI) for gfx950 with hipcc, in-tree.

Usage: python -m flint_amd.build   (or flint_amd.build.build())
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libflint_amd.so")
OBJDIR = os.path.join(HERE, "_build")
SOURCES = ["fl_quant.hip", "fl_decode.hip", "fl_sample.hip", "fl_probe.hip", "fl_tiled.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off",            # bf16 rounding points must match torch's op-by-op evaluation
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# per-source extra flags: the MFMA-dequant kernels keep their matrix-core results in VGPRs (the
# accumulation registers would cost a copy per result read by the vector ALUs)
EXTRA = {"fl_tiled.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src):
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    ext = build_torch_ext()
    if verbose:
        print(f"built {ext}")
    return OUT


TORCH_EXT = "_torch_ops"


def torch_ext_path():
    import sysconfig
    return os.path.join(HERE, TORCH_EXT + sysconfig.get_config_var("EXT_SUFFIX"))


def build_torch_ext():
    """The torch-extension binding (csrc/fl_torch.cpp: pybind11 ops over torch tensors) as
    flint_amd/_torch_ops*.so, linked against libflint_amd.so beside it. A host-only C++ file:
    it calls the C ABI and needs torch's headers, not HIP's."""
    import sysconfig
    import torch
    from torch.utils import cpp_extension
    out = torch_ext_path()
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"]]
    libs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
           os.path.join(CSRC, "fl_torch.cpp"), "-o", out + ".tmp",
           f"-DTORCH_EXTENSION_NAME={TORCH_EXT}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-deprecated-declarations",
           *[f"-I{i}" for i in incs], *[f"-L{l}" for l in libs], f"-L{HERE}",
           "-lflint_amd", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{l}" for l in libs]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{r.stderr[-4000:]}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
