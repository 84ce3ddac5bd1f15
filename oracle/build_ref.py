"""Build recipe for oracle/_ref -- TEST INFRASTRUCTURE ONLY.

Compiles the reference's dropout hash (reference @ None:
csrc/flash_attn_v100/fa_common.cuh:21-38, `hash_u32` and `dropout_keep`) with
hipcc for gfx950 into ``oracle/_ref/libfa2ref_hash.so``, wrapped by the
harness kernels of ``oracle/ref_hash_harness.hip``.  The GPU test
``tests/test_gpu_ref_hash.py`` compares its keep bits with the oracle's
restatement.

The source lines are taken from the reference file where it lies, at build
time: the text from the definition of ``hash_u32`` through the closing brace
of ``dropout_keep`` is written to a temporary directory outside the
repository, compiled, and deleted.  Nothing of the reference is kept in the
repository; only the built library goes to ``oracle/_ref/`` (git-ignored; it
travels to the GPU box with the other built libraries).  The rest of
fa_common.cuh includes <cuda_fp16.h>, which this image lacks, so the whole
header is not compiled and no stand-in header is written.

Run ``python oracle/build_ref.py``; ``__graft_entry__.build()`` calls
``build()`` when the reference tree is present.
"""
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_ref")
LIB = os.path.join(OUT_DIR, "libfa2ref_hash.so")
REF = os.environ.get("FA2_REFERENCE", "/root/reference")
HEADER = os.path.join(REF, "csrc", "flash_attn_v100", "fa_common.cuh")
HIPCC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")


def available():
    return os.path.isfile(HEADER)


def extract_hash_lines(text):
    """The lines from `__device__ __forceinline__ unsigned int hash_u32(` through
    the first line that is only `}` after the line defining `dropout_keep(`.
    Returns (first_line_number, lines); raises if the file no longer has that
    shape."""
    lines = text.split("\n")
    start = next(i for i, l in enumerate(lines) if re.match(r"\s*__device__ __forceinline__ unsigned int hash_u32\(", l))
    dk = next(i for i in range(start, len(lines)) if re.search(r"\bbool dropout_keep\(", lines[i]))
    end = next(i for i in range(dk, len(lines)) if lines[i].strip() == "}")
    block = lines[start:end + 1]
    body = "\n".join(block)
    if body.count("{") != body.count("}") or "#include" in body:
        raise RuntimeError(f"unexpected shape of {HEADER} lines {start + 1}-{end + 1}")
    return start + 1, block


def build(verbose=False):
    """Compile oracle/_ref/libfa2ref_hash.so; returns its path (None when the
    reference tree is absent, as on the GPU box)."""
    if not available():
        return None
    with open(HEADER) as f:
        first, block = extract_hash_lines(f.read())
    os.makedirs(OUT_DIR, exist_ok=True)
    tmpdir = tempfile.mkdtemp(prefix="fa2ref_")
    try:
        inc = os.path.join(tmpdir, "fa_common_hash_lines.inc")
        with open(inc, "w") as f:
            f.write(f'#line {first} "{HEADER}"\n' + "\n".join(block) + "\n")
        tmp = LIB + ".tmp"
        cmd = [HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-shared",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               f'-DFA2REF_HASH_LINES="{inc}"', os.path.join(HERE, "ref_hash_harness.hip"), "-o", tmp]
        proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"oracle/_ref build failed:\n{proc.stdout}")
        if verbose:
            print(f"compiled {HEADER}:{first}-{first + len(block) - 1}")
        os.replace(tmp, LIB)
    finally:
        shutil.rmtree(tmpdir, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv) or "reference tree absent: nothing built")
