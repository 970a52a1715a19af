"""CPU checks of the C ABI: the library loads and exports every symbol the
header declares, and the header declares every symbol the binding expects."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "talechime_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(tc_[a-z_0-9]+)\s*\(", src))


def test_header_matches_binding():
    from talechime_amd import _lib
    assert _declared() == set(_lib.EXPORTS)


def test_library_exports_every_symbol():
    from talechime_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libtalechime_hip.so not built")
    import torch  # noqa: F401  (same HIP runtime the product binds to)
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    lib.tc_abi_version.restype = ctypes.c_int
    assert lib.tc_abi_version() == 3


def _c_layout(struct: str, fields):
    """sizeof and offsetof of `struct` as gcc lays it out for the header."""
    import subprocess
    import tempfile
    lines = [f'printf("%zu\\n", sizeof({struct}));']
    lines += [f'printf("%zu\\n", offsetof({struct}, {f}));' for f in fields]
    prog = ("#include <stdio.h>\n#include <stddef.h>\n#include \"talechime_hip.h\"\n"
            "int main(void) {\n" + "\n".join(lines) + "\nreturn 0;\n}\n")
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(c, "w").write(prog)
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()
    return int(out[0]), [int(x) for x in out[1:]]


@pytest.mark.parametrize("cname,pyname", [("tc_sample_params", "SampleParams"), ("tc_verify_out", "VerifyOut")])
def test_struct_layout_matches_header(cname, pyname):
    from talechime_amd import _lib
    cls = getattr(_lib, pyname)
    names = [f[0] for f in cls._fields_]
    size, offs = _c_layout(cname, names)
    assert ctypes.sizeof(cls) == size
    assert [getattr(cls, n).offset for n in names] == offs
