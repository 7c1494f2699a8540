"""Build the gfx950 sampler library and the CPU oracle (test checker).

    python gguf-rs-cli_amd/build.py

Produces gguf-rs-cli_amd/libgs_sampler.so (HIP, --offload-arch=gfx950) and
oracle/liboracle.so.  This replaces the reference's build.rs shader step
(GLSL -> SPIR-V via shaderc, build.rs:24-43) with hipcc code objects.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgs_sampler.so")
ORACLE_DIR = os.path.join(ROOT, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: every f32 op is a single IEEE op, as in the Rust
# reference.  Packed-FP32 instructions are disabled for all HIP code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-function-calls=false",
    "-Wall", "-Wno-unused-function",
]
SOURCES = ["gs_kernels.hip", "gs_api.cpp", "gs_gemv.hip", "gs_decode.hip", "gs_tokens.cpp"]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build_library(verbose=False):
    objs = []
    for src in SOURCES:
        obj = os.path.join(CSRC, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC] + HIP_FLAGS + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
        out = _run(cmd)
        if verbose and out:
            print(out)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    for o in objs:
        os.remove(o)
    return LIB


def build_oracle():
    _run(["make", "-s", "-C", ORACLE_DIR, "-B", "liboracle.so"])
    return os.path.join(ORACLE_DIR, "liboracle.so")


def build_all(verbose=False):
    lib = build_library(verbose)
    orc = build_oracle()
    return lib, orc


if __name__ == "__main__":
    print(build_all(verbose="-v" in sys.argv))
