"""Build the gfx950 token-path libraries in-tree.

* ``libgraspo_tokpath.so`` -- the HIP kernels and the C ABI of
  ``include/graspo_tokpath.h`` (hipcc, --offload-arch=gfx950).
* ``_graspo_tokpath_ops.so`` -- the thin PyTorch extension that registers
  ``torch.ops.graspo_tokpath.*`` and calls the C ABI (host-only C++, g++
  against the installed torch headers).

Both land next to this file so they travel with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libgraspo_tokpath.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
EXT_NAME = "_graspo_tokpath_ops"

HIP_SOURCES = ["tokpath_logprob.hip", "tokpath_sampler.hip", "tokpath_sampler_fast.hip",
               "tokpath_loss.hip", "tokpath_decode.hip",
               "tokpath_narrow.hip", "tokpath_lmhead.hip"]
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build graspo_amd)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ...")


def build_hip(verbose: bool = False) -> str:
    """Compile the HIP sources into libgraspo_tokpath.so (always rebuilds)."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = _hipcc()
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    cmds, objs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        cmds.append([hipcc, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
        if verbose:
            print(" ".join(cmds[-1]))
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(_run, cmds))
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def ext_path() -> str:
    return os.path.join(HERE, EXT_NAME + ".so")


def build_ext(verbose: bool = False) -> str:
    """Compile the host-only torch extension (links libgraspo_tokpath.so)."""
    import torch.utils.cpp_extension as ce

    inc = ce.include_paths()
    torch_lib = os.path.join(os.path.dirname(ce.__file__), "..", "lib")
    torch_lib = os.path.abspath(torch_lib)
    out = ext_path()
    tmp = out + ".tmp"
    abi = int(getattr(__import__("torch")._C, "_GLIBCXX_USE_CXX11_ABI", 1))
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2", "-std=c++17", "-shared", "-fPIC",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=" + EXT_NAME,
        *[f"-I{p}" for p in inc],
        f"-I{os.path.join(REPO, 'include')}",
        os.path.join(CSRC, "torch_ops.cpp"),
        "-o", tmp,
        f"-L{HERE}", "-lgraspo_tokpath",
        f"-L{torch_lib}", "-lc10", "-ltorch_cpu", "-ltorch",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = False) -> None:
    build_hip(verbose)
    build_ext(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", LIB_PATH, "and", ext_path())
