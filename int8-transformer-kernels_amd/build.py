"""Build the gfx950 kernel library and the `int8_ext` torch binding in-tree.

    python build.py            # build everything that is out of date
    python build.py --force    # rebuild everything

Outputs (next to this file, git-ignored, shipped to the GPU box as files):
    libint8k.so                 — hand-written HIP kernels + the C ABI (include/int8k.h)
    int8_ext<EXT_SUFFIX>.so     — torch binding, plain C++ over the C ABI

No hipify step and no torch.utils.cpp_extension JIT: hipcc compiles the .hip
sources for gfx950 only, g++ compiles the binding against torch's headers.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

LIB_NAME = "libint8k.so"
CALIB_LIB_NAME = "libint8k_calib.so"
EXT_NAME = "int8_ext"

HIP_SOURCES = ["status.hip", "decode.hip", "mlp.hip", "prefill.hip", "quant.hip", "producer.hip",
               "noalloc.hip"]

# -packed-fp32-ops: keep v_pk_{add,mul,fma}_f32 out of the generated code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def lib_path() -> str:
    return os.path.join(PKG_DIR, LIB_NAME)


def ext_path() -> str:
    return os.path.join(PKG_DIR, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that notice is noise.
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _newer(target: str, deps: list[str]) -> bool:
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def _headers() -> list[str]:
    hs = [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    hs += [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    return hs


def build_lib(force: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    headers = _headers()
    objs, jobs = [], []
    for src in HIP_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        objs.append(o)
        if force or _newer(o, [s] + headers):
            jobs.append([HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", s, "-o", o])
    if jobs:
        with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
            list(ex.map(_run, jobs))
    out = lib_path()
    if force or jobs or _newer(out, objs):
        tmp = out + ".tmp"
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp,
              f"-Wl,-soname,{LIB_NAME}"])
        os.replace(tmp, out)
    return out


def build_calib(force: bool = False) -> str:
    """Roofline calibration kernels (bench only), a library of their own."""
    src = os.path.join(CSRC, "calib.hip")
    out = os.path.join(PKG_DIR, CALIB_LIB_NAME)
    if force or _newer(out, [src]):
        _run([HIPCC, *HIP_FLAGS, "-shared", src, "-o", out + ".tmp"])
        os.replace(out + ".tmp", out)
    return out


def build_ext(force: bool = False) -> str:
    import torch  # noqa: F401  (headers and libraries of the installed torch)
    from torch.utils import cpp_extension

    out = ext_path()
    src = os.path.join(CSRC, "int8_ext.cpp")
    if not (force or _newer(out, [src, lib_path()] + _headers())):
        return out
    torch_dir = os.path.dirname(torch.__file__)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INCLUDE,
                                            os.path.join(ROCM, "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-deprecated-declarations",
           *[f"-I{i}" for i in incs], src, "-o", out + ".tmp",
           f"-L{PKG_DIR}", "-l:" + LIB_NAME,
           f"-L{os.path.join(torch_dir, 'lib')}",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(torch_dir, 'lib')}"]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


def build(force: bool = False) -> None:
    build_lib(force)
    build_calib(force)
    build_ext(force)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("--lib-only", action="store_true")
    args = ap.parse_args()
    build_lib(args.force)
    build_calib(args.force)
    if not args.lib_only:
        build_ext(args.force)
    print("built:", lib_path(), "" if args.lib_only else ext_path())
    sys.exit(0)
