"""Build the gfx950 HIP library libs2x.so in-tree with hipcc.

    python hbd-siglip2.cpp_amd/build.py [--jobs N] [--asm]

Every HIP source is compiled with -ffp-contract=off (rounding points are
part of the numerical contract) and with packed-FP32 instruction selection
disabled.  The shared library lands next to this file.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libs2x.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = [
    "s2x_quant.hip",
    "s2x_gemm.hip",
    "s2x_attn.hip",
    "s2x_misc.hip",
    "s2x_naflex.hip",
    "s2x_static.hip",
    "s2x_abi.cpp",
    "s2x_encoders.cpp",
    "s2x_gguf.cpp",
    "siglip2_api.cpp",
    "siglip2_preproc.cpp",
]

COMMON = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def _compile(src, asm=False):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON]
    if src.endswith(".hip"):
        # MFMA results straight into VGPRs: the GEMM and attention kernels
        # post-process every MFMA tile on the VALU, and the default AGPR
        # destinations cost one v_accvgpr_read per element before each use
        cmd += ["-x", "hip", "-mllvm", "-amdgpu-mfma-vgpr-form"]
    cmd += ["-c", os.path.join(CSRC, src), "-o", obj]
    if asm and src.endswith(".hip"):
        cmd += ["-save-temps=obj"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    return src, r.returncode, out, obj


def build(jobs=None, asm=False, verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    objs = []
    failed = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, rc, out, obj in ex.map(lambda s: _compile(s, asm), SOURCES):
            if out.strip() and (verbose or rc):
                print(f"[{src}]\n{out}", file=sys.stderr)
            if rc:
                failed.append(src)
            objs.append(obj)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(failed))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


DRIVER_SRC = os.path.join(ROOT, "tests", "cpp", "drop_in_driver.cpp")
DRIVER = os.path.join(ROOT, "tests", "cpp", "drop_in_driver")


def build_driver():
    """The tests' C++ program over the drop-in classes (include/siglip2_*.h),
    linked against libs2x.so like a user's program would be."""
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"), DRIVER_SRC,
           "-L", HERE, "-ls2x", "-Wl,-rpath,$ORIGIN/../../hbd-siglip2.cpp_amd", "-o", DRIVER]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("driver build failed:\n" + r.stdout + r.stderr)
    return DRIVER


CLI_DIR = os.path.join(HERE, "cli")
BIN = os.path.join(HERE, "bin")
CLIS = {"siglip2-cli": "siglip2_cli.cpp", "siglip2-text-cli": "siglip2_text_cli.cpp"}


def build_cli():
    """The command-line encoders over the drop-in classes, into bin/."""
    os.makedirs(BIN, exist_ok=True)
    out = []
    for name, src in CLIS.items():
        exe = os.path.join(BIN, name)
        cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-I", os.path.join(ROOT, "include"),
               os.path.join(CLI_DIR, src), "-L", HERE, "-ls2x", "-Wl,-rpath,$ORIGIN/..",
               "-o", exe]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(f"{name} build failed:\n" + r.stdout + r.stderr)
        out.append(exe)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--asm", action="store_true", help="keep the gfx950 assembly")
    a = ap.parse_args()
    print(build(a.jobs, a.asm))
    print(build_driver())
    print(build_cli())
