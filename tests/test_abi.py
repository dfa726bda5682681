"""The C-ABI library without a GPU: it loads, exports every symbol that
include/strata_hip.h declares, and its host-only entry points behave.
No compute call is made here."""
import ctypes as C
import os
import re

import pytest

import strata_hip as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "strata_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = H.load_library()
    names = declared_symbols()
    assert names, "no declarations found"
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_mirror_lists_the_same_symbols():
    assert sorted(H.EXPORTS) == declared_symbols()


def test_abi_version_and_geometry():
    lib = H.load_library()
    assert lib.sh_abi_version() == 1
    assert H.quant_geometry(H.QuantType.Q8_0) == (32, 34)
    assert H.quant_geometry(H.QuantType.Q4_K) == (256, 144)
    assert H.quant_geometry(H.QuantType.Q5_K) == (256, 176)
    assert H.quant_geometry(H.QuantType.Q6_K) == (256, 210)
    assert H.quant_geometry(H.QuantType.IQ4_XS) == (256, 136)
    assert H.byte_size(H.QuantType.Q4_K, 12288) == 6912
    with pytest.raises(H.UnsupportedQuantError):
        H.quant_geometry(2)  # Q4_0: not on this path


def test_name_key_is_fnv1a():
    assert H.name_key("") == 0xCBF29CE484222325
    assert H.name_key("a") == 0xAF63DC4C8601EC8C


def test_null_arguments_are_rejected_without_a_device():
    lib = H.load_library()
    assert lib.sh_create(0, 0, None) == H.SH_ERR_INVALID_ARGUMENT
    assert lib.sh_gemv(None, None, None, 0, None, 0) == H.SH_ERR_INVALID_ARGUMENT
    assert "null" in H.last_error()
    assert lib.sh_destroy(None) == H.SH_OK


def test_create_reports_no_device_on_a_cpu_host():
    if H.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(H.NoDeviceError):
        H.HipBackend(0)


def test_dev_entry_points_validate_before_launch():
    # bad batch and unsupported types are refused on the host, no launch
    lib = H.load_library()
    assert lib.sh_gemv_dev(12, 0, None, 16, 256, None, None, 0, None) == H.SH_ERR_INVALID_ARGUMENT
    assert lib.sh_gemv_dev(2, 0, None, 16, 256, None, None, 1, None) == H.SH_ERR_UNSUPPORTED_QUANT
    assert lib.sh_gemv_dev(12, 0, None, 16, 200, None, None, 1, None) == H.SH_ERR_TRUNCATED
    assert lib.sh_dequant_dev(12, 0, None, 4, 256, None, None) == H.SH_ERR_INVALID_ARGUMENT


def test_tensor_byte_size_overflow_is_refused():
    # rows * (cols / 256) * 144 past 2^64: refused as an invalid argument, not
    # wrapped to a small size (which would admit a short buffer)
    lib = H.load_library()
    assert lib.sh_gemv_dev(12, 0, None, 1 << 60, 256 << 10, None, None, 1, None) == H.SH_ERR_INVALID_ARGUMENT
    assert "overflows" in H.last_error()
    # a product that fits is not an overflow (refused later, for the null pointers)
    assert lib.sh_gemv_dev(12, 0, None, 1 << 40, 256, None, None, 1, None) == H.SH_ERR_INVALID_ARGUMENT
    assert "overflows" not in H.last_error()


def test_header_is_plain_c_and_links(tmp_path):
    """include/strata_hip.h is a C99 header (what a cgo / bindgen / ctypes
    binding reads), and a C program calling through it links against the
    library: every declared symbol resolves at link time."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    header = os.path.join(root, "include", "strata_hip.h")
    names = declared_symbols()
    src = tmp_path / "use.c"
    src.write_text('#include "strata_hip.h"\n#include <stdio.h>\n'
                   'int main(void) {\n  void* p[] = {' + ", ".join(f"(void*)&{n}" for n in names) + '};\n'
                   '  printf("%d %d\\n", sh_abi_version(), (int)(sizeof p / sizeof p[0]));\n  return 0;\n}\n')
    lib = H.library_path()
    exe = tmp_path / "use"
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(header), str(src), "-o", str(exe),
                    lib, "-Wl,-rpath," + os.path.dirname(lib)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == [str(H.load_library().sh_abi_version()), str(len(names))]
