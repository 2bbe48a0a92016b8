"""The ctypes mirrors of the C ABI's descriptor structs have the C layout:
gcc compiles `include/qmoe.h` and prints sizeof / offsetof of every field,
which must equal the ctypes Structure's (a mismatch would hand the kernels
shifted pointers). CPU only."""

import os
import shutil
import subprocess

import pytest

from qmoe import _capi

INCLUDE = os.path.join(os.path.dirname(__file__), os.pardir, "include")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
@pytest.mark.parametrize("cname,pyname", [("qmoe_gemm_desc", "GemmDesc"), ("qmoe_moe_decode_desc", "DecodeDesc")])
def test_struct_layout_matches_c(tmp_path, cname, pyname):
    py = getattr(_capi, pyname)
    fields = [f[0] for f in py._fields_]
    lines = [f'printf("size %zu\\n", sizeof({cname}));']
    lines += [f'printf("{f} %zu\\n", offsetof({cname}, {f}));' for f in fields]
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "qmoe.h"\nint main(void) {\n  '
                   + "\n  ".join(lines) + "\n  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", INCLUDE, str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                       text=True).stdout.splitlines())
    assert int(out["size"]) == __import__("ctypes").sizeof(py)
    for f in fields:
        assert int(out[f]) == getattr(py, f).offset, f
