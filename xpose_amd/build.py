"""Build recipe for the native parts: libxpose.so (gfx950 HIP kernels + C ABI)
and oracle/liboracle.so (the CPU restatement used as the test checker).

Both are built in-tree so the shared objects travel with the source tree.
Usage: python -m xpose_amd.build [--lib-only | --oracle-only] [-v]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "xpose_amd", "csrc")
LIB = os.path.join(ROOT, "xpose_amd", "libxpose.so")
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")
OBJ_DIR = os.path.join(ROOT, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (the host pass warns
# that it does not know the feature; that is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Wno-unused-function", "-Xclang", "-target-feature", "-Xclang",
    "-packed-fp32-ops", "-munsafe-fp-atomics",
]

LIB_SOURCES = ["runtime.cpp", "synth.cpp", "matvec.hip", "transformer.hip", "sampling.hip",
               "sampling_chain.hip", "token_kernel.hip", "probe.hip", "batch_kernels.hip", "batch_step.hip",
               "batch.cpp", "gguf.cpp", "pack.cpp", "tokenizer.cpp", "repack.cpp", "native_quant.hip", "prefill_kernels.hip",
               "session_kernels.hip", "session.cpp"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd[:3])} ...")
    if verbose and (r.stdout or r.stderr):
        # Drop the known host-pass warning about the packed-fp32 feature.
        lines = [l for l in (r.stdout + r.stderr).splitlines()
                 if "packed-fp32-ops" not in l and l.strip()]
        if lines:
            print("\n".join(lines))


def build_lib(verbose: bool = False, extra: list[str] | None = None) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in LIB_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(OBJ_DIR, os.path.basename(s) + ".o")
        objs.append(o)
        lang = ["-x", "hip"] if s.endswith(".hip") else []
        cmds.append([HIPCC, *HIP_FLAGS, *(extra or []), *lang, "-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
          "-lpthread"], verbose)
    os.replace(tmp, LIB)
    return LIB


CLI_SRC = os.path.join(ROOT, "xpose_amd", "cli", "xpose_decode.cpp")
CLI_BIN = os.path.join(ROOT, "xpose_amd", "bin", "xpose_decode")


def build_cli(verbose: bool = False) -> str:
    """The C++ decode CLI over include/xpose.hpp (host code only, links
    libxpose.so, found next to it at run time through $ORIGIN)."""
    os.makedirs(os.path.dirname(CLI_BIN), exist_ok=True)
    tmp = CLI_BIN + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"), CLI_SRC,
          "-o", tmp, "-L", os.path.dirname(LIB), "-l:libxpose.so",
          "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath-link,/opt/rocm/lib"], verbose)
    os.replace(tmp, CLI_BIN)
    return CLI_BIN


def build_oracle(verbose: bool = False) -> str:
    # -ffp-contract=off: every a*b+c in the restatement rounds twice, exactly
    # as written; -march=x86-64-v3 so the object runs on any AVX2 host.
    tmp = ORACLE_LIB + ".tmp"
    _run(["gcc", "-O2", "-std=c11", "-fopenmp", "-ffp-contract=off", "-march=x86-64-v3",
          "-fPIC", "-shared", "-Wall", "-o", tmp, os.path.join(ORACLE_DIR, "oracle.c"),
          "-lm"], verbose)
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def build_all(verbose: bool = False) -> None:
    build_oracle(verbose)
    build_lib(verbose)
    build_cli(verbose)


if __name__ == "__main__":
    v = "-v" in sys.argv
    if "--oracle-only" in sys.argv:
        build_oracle(v)
    elif "--lib-only" in sys.argv:
        build_lib(v)
    else:
        build_all(v)
    if shutil.which("true"):
        print("built:", LIB if "--oracle-only" not in sys.argv else "", ORACLE_LIB)
