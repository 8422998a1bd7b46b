"""Build recipe for the oracle (test infrastructure, never the product).

    python oracle/build.py            # liboracle.so, plus _ref/ when the reference tree is present

Outputs:
  oracle/_build/liboracle.so  -- the C restatement (oracle.c, oracle_model.c)
  oracle/_ref/libref.so       -- the reference's own CPU routines, compiled from
                                 the reference sources where they lie:
                                 .auto/lfm3/q8_gemv_cpu.c (needs _Float16 -> ROCm clang)
                                 pulsar_arm/bonsai2/pq2_host.c
                                 pulsar_arm/bonsai2/bq1_cpu.c (its bq1_quant_row_i8: the
                                 Q8_K block rule, NEON-free, where fwd8.c's copy needs
                                 arm_neon.h)
Both directories are git-ignored and travel with the tree to a GPU machine.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REF_ROOT = "/root/reference"
CLANG = "/opt/rocm/llvm/bin/clang"
FLAGS = ["-O3", "-mavx2", "-mfma", "-ffp-contract=off", "-fPIC", "-shared"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)


def build_oracle():
    out_dir = os.path.join(HERE, "_build")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "liboracle.so")
    srcs = [os.path.join(HERE, f) for f in ("oracle.c", "oracle_model.c")]
    tmp = out + ".tmp"
    _run(["gcc", *FLAGS, "-fopenmp", "-std=c11", "-o", tmp, *srcs, "-lm"])
    os.replace(tmp, out)
    return out


def build_ref():
    """Compile the reference's CPU routines; returns the path or None when the
    reference tree is absent (a machine without it uses the prebuilt file)."""
    q8 = os.path.join(REF_ROOT, ".auto/lfm3/q8_gemv_cpu.c")
    pq2 = os.path.join(REF_ROOT, "pulsar_arm/bonsai2/pq2_host.c")
    bq1 = os.path.join(REF_ROOT, "pulsar_arm/bonsai2/bq1_cpu.c")
    if not (os.path.exists(q8) and os.path.exists(pq2) and os.path.exists(bq1)):
        return None
    out_dir = os.path.join(HERE, "_ref")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libref.so")
    tmp = out + ".tmp"
    omp_lib = "/opt/rocm/llvm/lib"
    _run([CLANG, *FLAGS, "-fopenmp", "-w", f'-DREF_Q8_CPU="{q8}"',
          "-I", os.path.dirname(pq2), "-o", tmp,
          os.path.join(HERE, "ref_shim.c"), pq2, bq1,
          "-L", omp_lib, f"-Wl,-rpath,{omp_lib}", "-lomp", "-lm"])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_oracle())
    print(build_ref())
    sys.exit(0)
