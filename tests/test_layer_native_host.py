"""CPU: the argument structs of soupk_layer_fwd / soupk_layer_bwd as include/soupk.h lays them
out (a C program built with gcc prints every field's offset and each struct's size) against
the ctypes structs testt_amd/layer_native.py fills."""

import ctypes
import os
import shutil
import subprocess

import pytest

from testt_amd import layer_native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STRUCTS = {"SoupkLayerDims": layer_native.LayerDims, "SoupkLayerFwd": layer_native.LayerFwd,
           "SoupkLayerBwd": layer_native.LayerBwd, "SoupkNf4Group": layer_native.Nf4Group,
           "SoupkLayerNf4": layer_native.LayerNf4}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is needed to lay out the header")
def test_struct_layouts_match_the_header(tmp_path):
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "soupk.h"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        cname, field, value = line.split()
        got[(cname, field)] = int(value)
    for cname, py in STRUCTS.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)
