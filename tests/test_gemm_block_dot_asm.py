"""The throughput GEMM writes its int8 block dot as inline assembly
(`v_mfma_i32_32x32x32_i8 ..., 0.15915494`: the accumulator operand as the
inline constant 1/2pi), which the compiler's hazard recognizer does not
see.  That is sound because the only reader of each block dot's result is
the conversion MFMA that takes it, register for register, as its
accumulator operand -- a dependency that needs no wait states (the compiler
itself issues two such builtins back to back).  This test compiles
s2x_gemm.hip to gfx950 assembly and checks, for every inline block dot,
that the first later instruction touching any of its result registers is
that conversion MFMA with exactly those registers as its accumulator; and,
as the reference for "no wait states", that the compiler issues the
builtin pair back to back."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "hbd-siglip2.cpp_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include"), "-I", CSRC,
         "-x", "hip", "-mllvm", "-amdgpu-mfma-vgpr-form", "--cuda-device-only", "-S"]

pytestmark = pytest.mark.skipif(not (os.path.exists(HIPCC) or shutil.which("hipcc")),
                                reason="hipcc is not installed")


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m[1]), int(m[2]) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m[1])} if m else set()


def _operands(line):
    parts = line.split(None, 1)
    if len(parts) < 2:
        return []
    return [t.strip() for t in parts[1].split(",")]


def _instructions(asm):
    for line in asm.splitlines():
        t = line.strip()
        if not t or t.startswith((";", ".")) or t.endswith(":"):
            continue
        yield t


def _first_toucher_ok(instrs, i, dst):
    """True if the first instruction after i that names a register of dst
    is a v_mfma_f32_32x32x8_f16 whose accumulator operand is exactly dst."""
    for t in instrs[i + 1:]:
        ops = _operands(t)
        used = set()
        for o in ops:
            used |= _regs(o)
        if used & dst:
            return t.startswith("v_mfma_f32_32x32x8_f16") and len(ops) >= 4 and _regs(ops[3]) == dst
    return False


@pytest.mark.timeout(600)
def test_inline_block_dots_feed_only_their_conversion(tmp_path):
    out = tmp_path / "gemm.s"
    r = subprocess.run([HIPCC, *FLAGS, os.path.join(CSRC, "s2x_gemm.hip"), "-o", str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    instrs = list(_instructions(out.read_text()))
    dots = [i for i, t in enumerate(instrs)
            if t.startswith("v_mfma_i32_32x32x32_i8") and "0.15915494" in t]
    assert dots, "no inline block dots in the throughput GEMM"
    bad = [instrs[i] for i in dots if not _first_toucher_ok(instrs, i, _regs(_operands(instrs[i])[0]))]
    assert not bad, f"{len(bad)} of {len(dots)} block dots have another first reader, e.g. {bad[0]}"


@pytest.mark.timeout(300)
def test_compiler_issues_the_dependent_pair_back_to_back(tmp_path):
    # the two builtins with the block dot's result as the conversion's
    # accumulator: nothing but memory-counter waits between them
    src = tmp_path / "pair.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "typedef int v4i __attribute__((ext_vector_type(4)));\n"
        "typedef int v16i __attribute__((ext_vector_type(16)));\n"
        "typedef float v16f __attribute__((ext_vector_type(16)));\n"
        "typedef _Float16 v4h __attribute__((ext_vector_type(4)));\n"
        "__global__ void k(const v4i *a, const v4i *b, const v4h *c, v16f *o) {\n"
        "  int t = threadIdx.x;\n"
        "  v4i x = a[t], y = b[t];\n"
        "  v4h p = c[t], q = c[t + 64];\n"
        "  v16i m = 0x3E22F983;\n"
        "  v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, m, 0, 0, 0);\n"
        "  o[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(p, q, __builtin_bit_cast(v16f, d), 0, 0, 0);\n"
        "}\n")
    out = tmp_path / "pair.s"
    r = subprocess.run([HIPCC, *FLAGS, str(src), "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    instrs = list(_instructions(out.read_text()))
    i = next(n for n, t in enumerate(instrs) if t.startswith("v_mfma_i32_32x32x32_i8"))
    j = next(n for n in range(i + 1, len(instrs)) if instrs[n].startswith("v_mfma"))
    # only memory-counter waits may sit between them: no hazard padding
    assert all(t.startswith("s_waitcnt") for t in instrs[i + 1:j]), instrs[i:j + 1]
    assert instrs[j].startswith("v_mfma_f32_32x32x8_f16"), instrs[i:j + 1]
    assert _regs(_operands(instrs[j])[3]) == _regs(_operands(instrs[i])[0])


def test_the_scan_rejects_other_first_readers():
    # the checker on made-up sequences: a VALU copy of the block dot's
    # result, a conversion whose accumulator only overlaps it, and the
    # accepted form
    dot = "v_mfma_i32_32x32x32_i8 v[2:17], v[20:23], v[24:27], 0.15915494"
    conv_ok = "v_mfma_f32_32x32x8_f16 v[2:17], v[30:31], v[32:33], v[2:17]"
    conv_part = "v_mfma_f32_32x32x8_f16 v[4:19], v[30:31], v[32:33], v[4:19]"
    copy = "v_mov_b32_e32 v40, v5"
    other = "v_add_u32_e32 v41, v42, v43"
    dst = _regs(_operands(dot)[0])
    assert _first_toucher_ok([dot, other, conv_ok], 0, dst)
    assert not _first_toucher_ok([dot, copy, conv_ok], 0, dst)
    assert not _first_toucher_ok([dot, conv_part], 0, dst)
    assert not _first_toucher_ok([dot, other], 0, dst)
