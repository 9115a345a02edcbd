"""The C-ABI library loads and exports every entry point include/drama3_moe.h declares (no GPU needed: nothing is
launched), and the Python binding knows each of them."""
import ctypes
import pathlib
import re
import subprocess

import pytest

from drama3 import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "drama3_moe.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(d3_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "d3_moe_a8" in names and "d3_last_error" in names


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert sorted(set(declared()) - set(_lib.SIGNATURES)) == []


def test_host_only_calls():
    lib = _lib.lib()
    assert lib.d3_version() >= 1
    assert lib.d3_moe_a8_workspace_bytes(16, 8, 2048, 768) > 0
    # argument errors come back as D3_EINVAL with a message, without touching a device
    rc = lib.d3_moe_a8(None, None)
    assert rc == -1 and b"null" in lib.d3_last_error()


@pytest.mark.parametrize("struct,cname", [(_lib.MoeA8Desc, "d3_moe_a8_desc"),
                                          (_lib.MoeA8PrefillDesc, "d3_moe_a8_prefill_desc")])
def test_descriptor_layout_matches_header(struct, cname, tmp_path):
    """Every field of the ctypes descriptor sits at the offset the C compiler gives it in the header, and the sizes
    agree: a field added to one side only shifts the rest and is caught here."""
    fields = [f[0] for f in struct._fields_]
    prog = tmp_path / "layout.c"
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {",
             f'  printf("size %zu\\n", sizeof({cname}));']
    lines += [f'  printf("{f} %zu\\n", offsetof({cname}, {f}));' for f in fields]
    lines += ["  return 0;", "}"]
    prog.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(prog)], check=True, capture_output=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                       text=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(struct)
    for f in fields:
        assert int(got[f]) == getattr(struct, f).offset, f


def test_grouped_switch_per_format():
    """moe_layer's switch to the grouped path (host logic): int8 and FP8 from 6 rows, W4A8 from 8, W6A8 from 9, and
    a row count past the fused kernel's 16 rows always grouped."""
    from drama3 import formats, moe
    assert moe.grouped_from_rows(formats.FMT_I8) == moe.GROUPED_FROM_ROWS == 6
    assert moe.grouped_from_rows(formats.FMT_F8) == 6
    assert moe.grouped_from_rows(formats.FMT_W4) == 8
    assert moe.grouped_from_rows(formats.FMT_W6) == 9
    assert all(moe.grouped_from_rows(f) <= moe.MAX_ROWS + 1 for f in range(4))
