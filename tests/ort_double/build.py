"""Builds tests/ort_double/libxm_ort_double.so: the custom-op layer of
xmetai-onnx-plugins_amd/csrc/ort compiled against the ONNX Runtime API double
beside this file, linked with the runtime double (ort_double.cpp) and the
operator library libxmetai_recurrent.so.  Test infrastructure: the tests load
it to register and run the operators as an ONNX Runtime session would.

    python tests/ort_double/build.py
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
PKG = os.path.join(ROOT, "xmetai-onnx-plugins_amd", "xmetai_onnx_plugins")
ORT_SRC = os.path.join(ROOT, "xmetai-onnx-plugins_amd", "csrc", "ort")
OUT = os.path.join(HERE, "libxm_ort_double.so")
SOURCES = [os.path.join(ORT_SRC, f) for f in ("register_op.cpp", "ops_ort.cpp", "softmax_cpu_ort.cpp")] + [
    os.path.join(HERE, "ort_double.cpp")]


def build() -> str:
    if not os.path.exists(os.path.join(PKG, "libxmetai_recurrent.so")):
        raise RuntimeError("libxmetai_recurrent.so is not built (python xmetai-onnx-plugins_amd/build.py)")
    rpath = os.path.relpath(PKG, HERE)
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Werror",
           "-I", HERE, "-I", os.path.join(ROOT, "include"), *SOURCES,
           "-L", PKG, "-lxmetai_recurrent", f"-Wl,-rpath,$ORIGIN/{rpath}", "-o", OUT + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("ORT double build failed:\n" + " ".join(cmd) + "\n" + r.stderr)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build())
    sys.exit(0)
