"""Build recipe for the native parts of op_plugin_amd (run in-tree, no JIT cache).

1. Every ``csrc/**/*.hip`` file outside ``csrc/calib`` is compiled for gfx950
   with hipcc and linked into ``op_plugin_amd/libqk_hip.so`` -- the C ABI of
   ``include/qk_abi.h``.
2. ``csrc/ops/npu_quant_ops.cpp`` (torch.ops.npu.* registration) is compiled
   with the host C++ compiler against torch's headers and linked against
   ``libqk_hip.so`` into ``op_plugin_amd/_npu_ops.so``.
3. ``csrc/calib/calibrate.hip`` (roofline calibration kernels for
   ``bench.py --calibrate``; not part of the op path) becomes
   ``op_plugin_amd/libqk_calib.so``.

Usage: ``python ascend-python_amd/build.py`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "op_plugin_amd")
OBJ = os.path.join(HERE, "_build")
ROOT = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-std=c++17", "-O3", "-fPIC",
    # every rounding point is written out (fmaf where fused is meant)
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    # no packed-fp32 instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd[:3])} ... {cmd[-1]}")
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    noise = [ln for ln in r.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln
             and "warning generated" not in ln]
    if verbose and noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build_hip(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(s for s in glob.glob(os.path.join(CSRC, "**", "*.hip"), recursive=True)
                  if os.sep + "calib" + os.sep not in s)
    objs = [os.path.join(OBJ, os.path.relpath(s, CSRC).replace(os.sep, "_") + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", s, "-o", o], verbose) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    lib = os.path.join(PKG, "libqk_hip.so")
    tmp = lib + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, lib)
    return lib


def build_ops(verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch.compiled_with_cxx11_abi())
    incs = [f"-I{p}" for p in cpp_extension.include_paths()] + [f"-I{os.path.join(ROCM, 'include')}",
                                                                 f"-I{sysconfig.get_paths()['include']}"]
    out = os.path.join(PKG, "_npu_ops.so")
    tmp = out + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_npu_ops",
           "-fvisibility=hidden", *incs, os.path.join(CSRC, "ops", "npu_quant_ops.cpp"),
           "-o", tmp, f"-L{PKG}", "-lqk_hip", f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build_calib(verbose: bool = False) -> str:
    lib = os.path.join(PKG, "libqk_calib.so")
    tmp = lib + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", tmp, os.path.join(CSRC, "calib", "calibrate.hip")], verbose)
    os.replace(tmp, lib)
    return lib


def build(verbose: bool = False) -> None:
    build_hip(verbose)
    build_ops(verbose)
    build_calib(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
