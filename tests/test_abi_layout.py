"""CPU: the Python mirrors of the C ABI's structs (treesa_gpu_amd/capi.py) have the header's layout.

A C program compiled with gcc from include/treesa_hip.h prints sizeof and offsetof of every field of
tsa_layout_t, tsa_config_t, tsa_select_t and tsa_trace_row_t; the ctypes structures and the trace-row numpy
dtype must agree field by field, so that a field added to the header without its mirror (or in another place)
fails here instead of shifting what the library reads.
"""
import ctypes
import os
import subprocess

import pytest

from treesa_gpu_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

MIRRORS = {
    "tsa_layout_t": capi.Layout,
    "tsa_config_t": capi.Config,
    "tsa_select_t": capi.Select,
}


def c_layout(tmp_path):
    fields = {name: [f for f, _ in cls._fields_] for name, cls in MIRRORS.items()}
    fields["tsa_trace_row_t"] = list(capi.TRACE_ROW.names)
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "treesa_hip.h"', "int main(void) {"]
    for name, fs in fields.items():
        lines.append(f'  printf("{name} size %zu\\n", sizeof({name}));')
        for f in fs:
            lines.append(f'  printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        name, field, v = line.split()
        got[(name, field)] = int(v)
    return got


def test_struct_mirrors_match_header(tmp_path):
    got = c_layout(tmp_path)
    for name, cls in MIRRORS.items():
        assert got[(name, "size")] == ctypes.sizeof(cls), name
        for f, _ in cls._fields_:
            assert got[(name, f)] == getattr(cls, f).offset, (name, f)
    assert got[("tsa_trace_row_t", "size")] == capi.TRACE_ROW.itemsize
    for f in capi.TRACE_ROW.names:
        assert got[("tsa_trace_row_t", f)] == capi.TRACE_ROW.fields[f][1], ("tsa_trace_row_t", f)


def test_a_missing_mirror_field_is_caught(tmp_path):
    """Planted on the Python side: a mirror without the header's last field is one int32 short."""
    class Short(ctypes.Structure):
        _fields_ = capi.Config._fields_[:-1]
    got = c_layout(tmp_path)
    assert got[("tsa_config_t", "size")] != ctypes.sizeof(Short)
    with pytest.raises(AssertionError):
        assert got[("tsa_config_t", "size")] == ctypes.sizeof(Short)
