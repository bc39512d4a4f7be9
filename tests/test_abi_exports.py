"""libs2x.so loads and exports every entry point include/*.h declares.
CPU only: nothing here touches a GPU."""
import ctypes
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "hbd-siglip2.cpp_amd", "libs2x.so")


def _declared_c_symbols():
    text = open(os.path.join(ROOT, "include", "s2x.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(s2x_[a-z0-9_]+)\s*\(", text))
    assert len(names) > 30
    return sorted(names)


def test_library_loads_and_exports_c_abi():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in _declared_c_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_cpp_api_symbols_exported():
    out = subprocess.run(["nm", "-DC", "--defined-only", LIB], capture_output=True,
                         text=True, check=True).stdout
    for sym in ["siglip2::VisionEncoder::encode(float const*, int, int, siglip2::Pooling, "
                "std::vector<float, std::allocator<float> >&)",
                "siglip2::VisionEncoder::load(std::__cxx11::basic_string<char, "
                "std::char_traits<char>, std::allocator<char> > const&, bool)",
                "siglip2::TextEncoder::encode(int const*, int, int const*, "
                "std::vector<float, std::allocator<float> >&)",
                "siglip2::TextEncoder::encode_batch(int const*, int, int, int const*, "
                "std::vector<float, std::allocator<float> >&)"]:
        assert sym in out, sym


def test_host_only_entry_points():
    import s2x
    assert s2x.version().startswith("s2x")
    assert s2x.lib.s2x_status_string(0) == b"ok"
    assert s2x.lib.s2x_weight_bytes(1152, 3456) >= 1152 * 3456 + 36 * 3456 * 2
    assert s2x.lib.s2x_weight_bytes(33, 1) == 0  # K not a multiple of 32
    ws = s2x.lib.s2x_mul_mat_workspace_size(4320, 1152, 729)
    assert ws >= 4320 * 1152 + 729 * 4320 + 729 * 135 * 4
    assert s2x.lib.s2x_attn_workspace_size(32, 729, 16, 72) > 0


def test_invalid_arguments_rejected_without_gpu():
    import s2x
    # argument checks run before any HIP call
    st = s2x.lib.s2x_quantize_q8_1(None, 1152, 4, 1152, 1000, None, None, None)
    assert st == 1 and b"bad shape" in s2x.lib.s2x_last_error()
    st = s2x.lib.s2x_mul_mat_q8_0_f32(None, 4320, 1152, None, 4400, 4400, 2, None, None, 0, None)
    assert st == 1
    out = ctypes.c_void_p()
    assert s2x.lib.s2x_vision_create(None, ctypes.byref(out)) == 1
