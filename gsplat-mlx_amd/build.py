"""Build the MI355X splatting chain in-tree.

Outputs (into gsplat-mlx_amd/gsplat_core/):
  libgsplat_hip.so   hand-written gfx950 HIP kernels + the C ABI (include/gsplat_hip.h)
  libgsplat_core.so  C++ operator API (namespace gsplat_core, at::Tensor), calls the C ABI
  _gsplat_core*.so   Python module with the reference binding's surface

Every HIP file is compiled with packed-FP32 instruction selection disabled
and FMA contraction off (kernels round like the reference's float32 CPU
loops: contraction turns cancellation-prone gradient elements ~1e-3 relative
away from them). GRADIENT_ONLY files compute only gradients (held to a
relative tolerance) and also use the fast float32 division / square root
(about 1 ulp; 2 us of the projection backward at a million Gaussians). Run
`python gsplat-mlx_amd/build.py` or `__graft_entry__.build()`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "gsplat_core")
OBJ = os.path.join(HERE, "_build")
HIP_SRC = os.path.join(HERE, "csrc", "hip")
CORE_SRC = os.path.join(HERE, "csrc", "core")
BIND_SRC = os.path.join(HERE, "csrc", "binding")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = os.environ.get("GSPLAT_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = ["common", "quat_scale_to_covar", "projection", "projection_bwd", "spherical_harmonics", "scan",
               "intersect", "bucket", "radix_sort", "rasterize", "training_glue", "image_loss"]
GRADIENT_ONLY = {"projection_bwd"}
CORE_SOURCES = ["gsplat_quat_scale_to_covar", "gsplat_projection", "gsplat_spherical_harmonics",
                "gsplat_intersect", "gsplat_rasterize", "gsplat_training_glue", "gsplat_render"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(line for line in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in line)
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{msg}")
    return r


def _torch_flags():
    import torch
    import torch.utils.cpp_extension as ce

    inc = ce.include_paths() + [sysconfig.get_paths()["include"], os.path.join(ROCM, "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-fPIC", "-std=c++17", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1",
              "-DUSE_ROCM=1", "-Wno-deprecated-declarations"] + [f"-I{p}" for p in inc]
    libdir = ce.library_paths()[0]
    return cflags, libdir


def build(verbose: bool = False, jobs: int | None = None) -> None:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(OUT, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    inc = [f"-I{os.path.join(ROOT, 'include')}", f"-I{HIP_SRC}"]

    hip_objs = [os.path.join(OBJ, f"{s}.hip.o") for s in HIP_SOURCES]
    cflags, torch_lib = _torch_flags()
    core_inc = [f"-I{os.path.join(CORE_SRC, 'include')}", f"-I{CORE_SRC}", f"-I{os.path.join(ROOT, 'include')}"]
    core_objs = [os.path.join(OBJ, f"{s}.o") for s in CORE_SOURCES]
    bind_obj = os.path.join(OBJ, "binding.o")
    bind_flags = ["-DTORCH_EXTENSION_NAME=_gsplat_core", "-DTORCH_API_INCLUDE_EXTENSION_H", "-fvisibility=hidden"]

    jobs_list = []
    for s, o in zip(HIP_SOURCES, hip_objs):
        flags = list(HIPCC_FLAGS)
        if s in GRADIENT_ONLY:
            flags = flags + ["-fno-hip-fp32-correctly-rounded-divide-sqrt"]
        jobs_list.append(["hipcc", *flags, *inc, "-c", os.path.join(HIP_SRC, f"{s}.hip"), "-o", o])
    for s, o in zip(CORE_SOURCES, core_objs):
        jobs_list.append(["g++", *cflags, *core_inc, "-c", os.path.join(CORE_SRC, f"{s}.cpp"), "-o", o])
    jobs_list.append(["g++", *cflags, *bind_flags, *core_inc, "-c", os.path.join(BIND_SRC, "binding.cpp"),
                      "-o", bind_obj])
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs_list))

    lib_hip = os.path.join(OUT, "libgsplat_hip.so")
    _run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib_hip + ".tmp", *hip_objs,
          "-Wl,-soname,libgsplat_hip.so"], verbose)
    os.replace(lib_hip + ".tmp", lib_hip)

    torch_libs = [f"-L{torch_lib}", f"-Wl,-rpath,{torch_lib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip",
                  "-ltorch", "-lamdhip64"]
    lib_core = os.path.join(OUT, "libgsplat_core.so")
    _run(["g++", "-shared", "-fPIC", "-o", lib_core + ".tmp", *core_objs, f"-L{OUT}", "-lgsplat_hip",
          "-Wl,-rpath,$ORIGIN", "-Wl,-soname,libgsplat_core.so", *torch_libs], verbose)
    os.replace(lib_core + ".tmp", lib_core)

    ext = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    mod = os.path.join(OUT, "_gsplat_core" + ext)
    _run(["g++", "-shared", "-fPIC", "-o", mod + ".tmp", bind_obj, f"-L{OUT}", "-lgsplat_core", "-lgsplat_hip",
          "-Wl,-rpath,$ORIGIN", *torch_libs, "-ltorch_python"], verbose)
    os.replace(mod + ".tmp", mod)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built:", ", ".join(sorted(f for f in os.listdir(OUT) if f.endswith(".so"))))
