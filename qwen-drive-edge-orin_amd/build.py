"""Build the gfx950 gated-delta-rule library and its torch extension in-tree.

Outputs (next to this file, under gdn_hip/):
  libgdn_hip.so                      C ABI (include/gdn_hip.h), hipcc, gfx950
  deltanet_chunk_hip<EXT_SUFFIX>     torch extension over that C ABI (g++)

Run ``python qwen-drive-edge-orin_amd/build.py`` (or call ``build()``).  Both
steps run without a GPU: hipcc cross-compiles the device code.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT = PKG_ROOT / "gdn_hip"
INCLUDE = REPO / "include"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["gdn_prefill.hip", "gdn_decode.hip", "gated_rmsnorm.hip", "causal_conv1d.hip",
               "stream_probe.hip"]
LIB_NAME = "libgdn_hip.so"
EXT_NAME = "deltanet_chunk_hip"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed fp32 VALU ops stay off (hipcc flag; the host pass warns, harmlessly)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the scan scales and converts its state
    # accumulators with VALU every chunk, which AGPR accumulators would turn
    # into accvgpr read / write round trips
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_lib() -> Path:
    out = OUT / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    _run([f"{ROCM}/bin/hipcc", *HIPCC_FLAGS, f"-I{INCLUDE}",
          *[str(CSRC / s) for s in HIP_SOURCES], "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_ext() -> Path:
    import torch
    import torch.utils.cpp_extension as ce
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = OUT / f"{EXT_NAME}{suffix}"
    tmp = OUT / f"{EXT_NAME}.so.tmp"
    incs = ce.include_paths(device_type="cuda") + [sysconfig.get_paths()["include"],
                                                   pybind11.get_include(), str(INCLUDE)]
    libdirs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DHIPBLAS_V2",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in incs],
           str(CSRC / "torch_binding.cpp"),
           f"-L{OUT}", "-lgdn_hip",
           *[f"-L{p}" for p in libdirs],
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
           "-lamdhip64",
           "-Wl,-rpath,$ORIGIN",
           "-o", str(tmp)]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build() -> None:
    OUT.mkdir(exist_ok=True)
    build_lib()
    build_ext()


if __name__ == "__main__":
    build()
    sys.exit(0)
