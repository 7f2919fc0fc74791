"""Build the MI355X W4A16 library and its PyTorch binding in-tree.

    python w4a16-gemm_amd/build.py            # builds both
    python w4a16-gemm_amd/build.py --lib      # only libw4a16_hip.so

Outputs (next to this file, git-ignored, shipped to the GPU box with the tree):
  libw4a16_hip.so              hipcc --offload-arch=gfx950: kernels + C ABI (include/w4a16.h)
  w4a16_opt<EXT_SUFFIX>        host-compiler (g++) PyTorch extension linking libw4a16_hip.so
                               through an $ORIGIN rpath; import it as `w4a16_opt`.
  w4a16_ext<EXT_SUFFIX>        the same for the baseline GEMV module `w4a16_ext`.
  libw4a16_bwprobe.so          bandwidth probes of measure_bw.py.
  libw4a16_hip_stamps.so       the same library built with -DW4A16_WAVE_STAMPS: the decode ring
                               kernel records per-wave timestamps (wave_timeline.py); never
                               loaded by the op, the tests' GEMM calls or bench.py.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
LIB = os.path.join(HERE, "libw4a16_hip.so")
EXT = os.path.join(HERE, "w4a16_opt" + sysconfig.get_config_var("EXT_SUFFIX"))
EXT_GEMV = os.path.join(HERE, "w4a16_ext" + sysconfig.get_config_var("EXT_SUFFIX"))

# gfx950 only; packed-fp32 VALU ops disabled for all device code (-packed-fp32-ops).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "target-feature" not in l)
    if out.strip():
        print(out, flush=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


# Sources of libw4a16_hip.so with their extra flags.  The wide prefill kernel is scheduled with
# the max-memory-clause strategy: with the default strategy its 128 MFMA accumulators are rotated
# through register copies inside the main loop (see the header of w4a16_prefill_wide.hip).  The
# GEMM and GEMV kernels' units preload the first 16 dwords of kernel arguments into SGPRs (gfx950
# kernel argument preloading; the compiler adds an entry that loads them itself where the firmware
# does not preload), so the kernels start their loads without an s_load round trip.
SOURCES = [
    ("w4a16_kernels.hip", ["-mllvm", "-amdgpu-kernarg-preload-count=16"]),
    ("w4a16_prefill_wide.hip", ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause",
                                "-mllvm", "-amdgpu-kernarg-preload-count=16"]),
    ("w4a16_quantize.hip", []),
    ("w4a16_gemv.hip", ["-mllvm", "-amdgpu-kernarg-preload-count=16"]),
    ("w4a16_plan.cpp", []),
]


def compile_flags(src: str) -> list[str]:
    """hipcc flags (without -c/-o) of one library source, also used by the assembly tests."""
    extra = dict(SOURCES)[src]
    return [*HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}"]


STAMPS_OBJ = "w4a16_kernels_stamps.o"


def build_lib(with_stamps: bool = False) -> str:
    """libw4a16_hip.so; with_stamps also compiles the instrumented kernels object of
    build_stamps in the same parallel pool (the two kernels files are the long poles)."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, src.rsplit(".", 1)[0] + ".o") for src, _ in SOURCES]
    cmds = [[hipcc, *compile_flags(src), "-c", os.path.join(CSRC, src), "-o", obj]
            for (src, _), obj in zip(SOURCES, objs)]
    if with_stamps:
        cmds.insert(1, [hipcc, *compile_flags("w4a16_kernels.hip"), "-DW4A16_WAVE_STAMPS", "-c",
                        os.path.join(CSRC, "w4a16_kernels.hip"), "-o", os.path.join(objdir, STAMPS_OBJ)])
    # the translation units compile independently: in parallel (the kernels file is the long pole)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(cmds)) as pool:
        jobs = [pool.submit(_run, cmd) for cmd in cmds]
        for job in jobs:
            job.result()
    tmp = LIB + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


PROBE = os.path.join(HERE, "libw4a16_bwprobe.so")
STAMPS = os.path.join(HERE, "libw4a16_hip_stamps.so")


def build_stamps() -> str:
    """libw4a16_hip_stamps.so: the kernels file built with -DW4A16_WAVE_STAMPS (by
    build_lib(with_stamps=True), which must have run first), linked with build_lib's other objects."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objdir = os.path.join(HERE, "_build")
    kobj = os.path.join(objdir, STAMPS_OBJ)
    objs = [kobj] + [os.path.join(objdir, src.rsplit(".", 1)[0] + ".o") for src, _ in SOURCES[1:]]
    tmp = STAMPS + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, STAMPS)
    return STAMPS


def build_probe() -> str:
    """The streaming-read probe of measure_bw.py (a separate tool library, not the GEMM ABI)."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = PROBE + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, "-shared", os.path.join(CSRC, "bw_probe.hip"), "-o", tmp])
    os.replace(tmp, PROBE)
    return PROBE


def build_ext(name: str = "w4a16_opt", source: str = "w4a16_torch.cpp", out: str = EXT) -> str:
    import torch.utils.cpp_extension as ce
    import torch

    cxx = os.environ.get("CXX", "g++")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [INCLUDE, CSRC, *ce.include_paths(), sysconfig.get_paths()["include"], os.path.join(ROCM, "include")]
    libdirs = [*ce.library_paths(), os.path.join(ROCM, "lib"), HERE]
    tmp = out + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-DTORCH_EXTENSION_NAME={name}",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-Wno-deprecated-declarations",
           *[f"-I{p}" for p in incs],
           os.path.join(CSRC, source),
           *[f"-L{p}" for p in libdirs],
           "-lw4a16_hip", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
           "-lamdhip64", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    _run(cmd)
    os.replace(tmp, out)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--lib", action="store_true", help="only build libw4a16_hip.so")
    a = ap.parse_args(argv)
    build_lib(with_stamps=not a.lib)
    if not a.lib:
        with concurrent.futures.ThreadPoolExecutor(max_workers=4) as pool:
            jobs = [pool.submit(build_stamps), pool.submit(build_probe), pool.submit(build_ext),
                    pool.submit(build_ext, "w4a16_ext", "w4a16_ext_torch.cpp", EXT_GEMV)]
            for job in jobs:
                job.result()
    return 0


if __name__ == "__main__":
    sys.exit(main())
