"""Build libtiermm.so in-tree for gfx950 (hipcc for the kernels, g++ for host-only code).

Run ``python -m tier_amd.build`` or call ``build()``; ``__graft_entry__.build()``
calls it.  Objects go to ``tier_amd/_build/``; the library to ``tier_amd/libtiermm.so``,
and bench.py's measurement kernels (probe.hip) to ``tier_amd/libtiermm_probe.so``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libtiermm.so")
# measurement kernels for bench.py only (the plain-read floor and the fp16 MFMA ceiling)
PROBE_LIB = os.path.join(HERE, "libtiermm_probe.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_SOURCES = ["dequant.hip", "qgemv.hip", "qgemv_q4k.hip", "qgemv_q4k_ws.hip", "qgemv_q6k.hip", "qgemm_fused.hip", "x3.hip",
               "noalloc.hip", "host_dequant.hip", "chat_ops.hip"]
CXX_SOURCES = ["api.cpp", "quantize.cpp", "tq.cpp", "chat.cpp"]

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 are generated (hipcc's host pass
# warns that it does not know the feature; harmless).
# -amdgpu-kernarg-preload-count=16: the first 16 argument dwords arrive in SGPRs when
# a wave starts (firmware without preload runs the s_load prologue the compiler adds
# ahead of the entry point), so the first loads of a kernel leave ~0.2 us earlier:
# q4_K 13824x5120 decode 8.52 -> 8.34 us, 5120x5120 5.77 -> 5.63 us.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-munsafe-fp-atomics",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-mllvm", "-amdgpu-kernarg-preload-count=16",
             "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]
# The quantizer must not fuse fp32 expressions (byte parity with the reference).
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-pthread", "-D__HIP_PLATFORM_AMD__",
             "-I", os.path.join(ROCM, "include"), "-Wall"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    jobs = []
    for src in HIP_SOURCES:
        obj = os.path.join(OUT_DIR, src + ".o")
        jobs.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
    for src in CXX_SOURCES:
        obj = os.path.join(OUT_DIR, src + ".o")
        jobs.append(["g++"] + CXX_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 4)) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    objs = [os.path.join(OUT_DIR, s + ".o") for s in HIP_SOURCES + CXX_SOURCES]
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp] + objs +
         ["-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-pthread", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, LIB)
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC] + HIP_FLAGS + ["-shared", "-o", tmp, os.path.join(CSRC, "probe.hip")])
    os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
