"""In-tree build of the gfx950 FMHA forward library, its bench CLI and the CPU oracle.

    python -m fmha_native_amd.build          # or: python fmha_native_amd/build.py

Outputs (git-ignored, but shipped to the GPU box with the tree):
  fmha_native_amd/libfmha_native_amd.so   kernels + C-ABI launcher + input generators
  fmha_native_amd/bench_fmha_fwd          the timing CLI
  oracle/liboracle.so                     CPU oracle (test infrastructure only)

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
import os
import shutil
import subprocess
import sys
import tempfile

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
ORACLE = os.path.join(ROOT, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

LIB = os.path.join(PKG, "libfmha_native_amd.so")
BENCH = os.path.join(PKG, "bench_fmha_fwd")
ORACLE_LIB = os.path.join(ORACLE, "liboracle.so")


def _run_all(cmds, verbose):
    procs = []
    for cmd in cmds:
        if verbose:
            print("+", " ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for cmd, p in procs:
        out, _ = p.communicate()
        # hipcc's host pass does not know the gfx feature; that warning is noise
        lines = [l for l in out.splitlines() if "not a recognized feature" not in l]
        if p.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        elif verbose and lines:
            print("\n".join(lines))
    if failed:
        msg = "\n\n".join(f"$ {' '.join(c)}\n{o}" for c, o in failed)
        raise RuntimeError(f"build failed:\n{msg}")


def build_oracle(verbose=False):
    """CPU oracle: plain C, OpenMP, no FMA contraction (bit-stable arithmetic)."""
    cmd = ["gcc", "-O3", "-mavx2", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared", "-std=c11",
           os.path.join(ORACLE, "fmha_oracle.c"), "-o", ORACLE_LIB + ".tmp", "-lm"]
    _run_all([cmd], verbose)
    os.replace(ORACLE_LIB + ".tmp", ORACLE_LIB)


def build(verbose=False):
    with tempfile.TemporaryDirectory(prefix="fmha_build_") as tmp:
        objs = {
            "kernel": os.path.join(tmp, "fmha_fwd_kernel.o"),
            "api": os.path.join(tmp, "fmha_fwd_api.o"),
            "merge": os.path.join(tmp, "fmha_merge.o"),
            "noalloc": os.path.join(tmp, "fmha_noalloc.o"),
            "runner": os.path.join(tmp, "runner.o"),
        }
        _run_all([
            [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, "fmha_fwd_kernel.hip"), "-o", objs["kernel"]],
            [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, "fmha_fwd_api.hip"), "-o", objs["api"]],
            [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, "fmha_merge.hip"), "-o", objs["merge"]],
            [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, "fmha_noalloc.hip"), "-o", objs["noalloc"]],
            ["g++", "-O3", "-fopenmp", "-fPIC", "-std=c++17", f"-I{CSRC}", "-c",
             os.path.join(CSRC, "runner.cpp"), "-o", objs["runner"]],
            ["gcc", "-O3", "-mavx2", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared", "-std=c11",
             os.path.join(ORACLE, "fmha_oracle.c"), "-o", ORACLE_LIB + ".tmp", "-lm"],
        ], verbose)
        os.replace(ORACLE_LIB + ".tmp", ORACLE_LIB)
        tmp_lib = os.path.join(tmp, "libfmha_native_amd.so")
        _run_all([[HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", objs["kernel"], objs["api"], objs["merge"], objs["noalloc"], objs["runner"],
                   "-lgomp", "-o", tmp_lib]], verbose)
        shutil.copyfile(tmp_lib, LIB + ".tmp")
        os.replace(LIB + ".tmp", LIB)
        tmp_bench = os.path.join(tmp, "bench_fmha_fwd")
        _run_all([[HIPCC, *HIP_FLAGS, os.path.join(CSRC, "bench_fmha_fwd.cpp"), f"-L{PKG}", "-lfmha_native_amd",
                   "-Wl,-rpath,$ORIGIN", "-o", tmp_bench]], verbose)
        shutil.copyfile(tmp_bench, BENCH + ".tmp")
        os.chmod(BENCH + ".tmp", 0o755)
        os.replace(BENCH + ".tmp", BENCH)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", LIB, BENCH, ORACLE_LIB)
