"""The C-ABI library as the header declares it (no GPU needed, no compute calls)."""

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dspine_verify.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)  # drop comments
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\s*\*)\s+(dsv_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for required in ("dsv_verify", "dsv_verify_workspace_bytes", "dsv_greedy_verify",
                     "dsv_greedy_workspace_bytes", "dsv_topk", "dsv_topk_workspace_bytes",
                     "dsv_uniforms", "dsv_last_error", "dsv_device_count", "dsv_profile_events",
                     "dsv_adjust_logits", "dsv_adjust_history", "dsv_logits_padding", "dsv_window_index",
                     "dsv_target_probs", "dsv_compress", "dsv_accept_chain", "dsv_sample_chain",
                     "dsv_pack_joint"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from dspine_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_lib.EXPORTS) == set(declared_functions())


@pytest.mark.parametrize("cls_name, c_name", [("VerifyArgs", "dsv_verify_args"), ("ChainArgs", "dsv_chain_args"),
                                              ("FactorArgs", "dsv_factor_args")])
def test_args_struct_layout_matches_c(tmp_path, cls_name, c_name):
    """ctypes field offsets == offsetof() of the C struct compiled by gcc."""
    from dspine_amd import _lib

    cls = getattr(_lib, cls_name)
    names = [f[0] for f in cls._fields_]
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "dspine_verify.h"', "int main(void) {",
             f'  printf("%zu\\n", sizeof({c_name}));']
    lines += [f'  printf("%zu\\n", offsetof({c_name}, {n}));' for n in names]
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert out[0] == ctypes.sizeof(cls)
    assert out[1:] == [getattr(cls, n).offset for n in names]
