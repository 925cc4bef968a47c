"""Builds the gfx950 shared library ``libxmetai_recurrent.so`` in-tree.

    python xmetai-onnx-plugins_amd/build.py [--jobs N] [--ort-include DIR --ort-lib DIR]

Every HIP and C++ source under ``csrc/`` is compiled with hipcc for gfx950
(objects under ``_build/``) and linked into
``xmetai_onnx_plugins/libxmetai_recurrent.so``, which exports the C ABI of
``include/xmetai_recurrent.h``.  ``csrc/probe/hbm_stream.hip`` becomes
``libxm_hbm_probe.so``, the streaming kernels bench.py times for the
achievable HBM bandwidth (not part of the operator library).  When ONNX Runtime headers are available
(``--ort-include`` or ``ORT_INCLUDE_DIR``), the custom-op layer under
``csrc/ort/`` is built as ``libxmetai_onnx_plugins_ort.so`` (exports
``RegisterCustomOps``, ``include/xmetai_onnx_plugins_ort.h``) on top of it.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
PKG = os.path.join(HERE, "xmetai_onnx_plugins")
LIB = os.path.join(PKG, "libxmetai_recurrent.so")
ORT_LIB = os.path.join(PKG, "libxmetai_onnx_plugins_ort.so")
PROBE_LIB = os.path.join(PKG, "libxm_hbm_probe.so")   # benchmark-only HBM streaming probe

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall",
    f"--offload-arch={ARCH}",
    # Packed fp32 (v_pk_*_f32) stays disabled for every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the GDN-2 chunk recurrence reads
    # every product with VALU code, which AGPR accumulators would route
    # through v_accvgpr_read copies (4 x 4096 x 16 heads: 0.646 -> 0.622 ms).
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-I", INCLUDE, "-I", CSRC,
]

SOURCES = [
    "xm_runtime.hip",
    "selective_scan.hip",
    "selective_scan_seg.hip",
    "gated_deltanet2.hip",
    "gated_deltanet2_chunk.hip",
    "gated_deltanet2_noalloc.hip",
    "mamba3_siso.hip",
    "mamba3_siso_chunk.hip",
    "selective_scan_host.cpp",
    "gated_deltanet2_host.cpp",
    "mamba3_siso_host.cpp",
    "softmax_cpu.cpp",
]

ORT_SOURCES = [
    "ort/register_op.cpp",
    "ort/ops_ort.cpp",
    "ort/softmax_cpu_ort.cpp",
]


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD, src.replace("/", "_") + ".o")
    path = os.path.join(CSRC, src)
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *COMMON, *extra, *lang, "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line.
    noise = "not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs: int | None = None, ort_include: str | None = None, ort_lib: str | None = None,
          verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, []), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True, capture_output=not verbose)
    os.replace(tmp, LIB)

    probe_obj = _compile("probe/hbm_stream.hip", [])
    tmp = PROBE_LIB + ".tmp"
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, probe_obj], check=True,
                   capture_output=not verbose)
    os.replace(tmp, PROBE_LIB)

    ort_include = ort_include or os.environ.get("ORT_INCLUDE_DIR")
    ort_lib = ort_lib or os.environ.get("ORT_LIB_DIR")
    if ort_include and os.path.exists(os.path.join(ort_include, "onnxruntime_c_api.h")):
        extra = ["-I", ort_include]
        with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            ort_objs = list(ex.map(lambda s: _compile(s, extra), ORT_SOURCES))
        link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", ORT_LIB, *ort_objs,
                "-L", PKG, "-lxmetai_recurrent", "-Wl,-rpath,$ORIGIN"]
        if ort_lib:
            link += ["-L", ort_lib, "-lonnxruntime"]
        subprocess.run(link, check=True, capture_output=not verbose)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--ort-include", default=None)
    ap.add_argument("--ort-lib", default=None)
    ap.add_argument("--clean", action="store_true")
    args = ap.parse_args()
    if args.clean and os.path.isdir(BUILD):
        shutil.rmtree(BUILD)
    print(build(args.jobs, args.ort_include, args.ort_lib, verbose=True))


if __name__ == "__main__":
    main()
