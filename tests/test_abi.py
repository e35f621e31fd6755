"""The C-ABI library: it loads, exports every declared symbol, and its structs match (CPU).

No compute entry point is called here: only ``cb_abi_version``,
``cb_last_error`` and argument validation that fails before any HIP call.
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess

import pytest

from cachebridge_amd import _lib

from .conftest import ROOT

HEADER = ROOT / "include" / "cachebridge_hip.h"


def _declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^[A-Za-z_][\w \*]*?\b(cb_\w+)\s*\(", text, flags=re.M))


def _header_defines() -> dict[str, int]:
    out = {}
    for name, value in re.findall(r"^#define\s+(CB_\w+)\s+\(?(-?\d+)\)?", HEADER.read_text(), re.M):
        out[name] = int(value)
    return out


@pytest.fixture(scope="module")
def lib(built_library):
    return _lib.load()


def test_header_declares_exactly_the_bound_symbols():
    assert _declared_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib, built_library):
    for name in _declared_functions():
        assert hasattr(lib, name), name
    nm = shutil.which("nm")
    if nm:
        dyn = subprocess.run([nm, "-D", "--defined-only", str(built_library)],
                             capture_output=True, text=True, check=True).stdout
        exported = set(re.findall(r"\bT (cb_\w+)$", dyn, re.M))
        assert _declared_functions() <= exported


def test_abi_version_and_constants(lib):
    assert lib.cb_abi_version() == 1
    defines = _header_defines()
    assert defines["CB_ABI_VERSION"] == 1
    for name, value in defines.items():
        if name == "CB_ABI_VERSION":
            continue
        assert getattr(_lib, name) == value, name


def _c_layout(struct: str, fields: list[str]) -> list[int]:
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    return _compile_and_run(gcc, struct, fields)


def _compile_and_run(gcc, struct, fields):
    import tempfile
    from pathlib import Path

    lines = [f'printf("%zu\\n", sizeof({struct}));']
    lines += [f'printf("%zu\\n", offsetof({struct}, {f}));' for f in fields]
    src = ("#include <stddef.h>\n#include <stdio.h>\n#include \"cachebridge_hip.h\"\n"
           "int main(void) {\n" + "\n".join(lines) + "\nreturn 0;\n}\n")
    with tempfile.TemporaryDirectory() as tmp:
        c = Path(tmp) / "layout.c"
        exe = Path(tmp) / "layout"
        c.write_text(src)
        subprocess.run([gcc, "-std=c11", "-I", str(HEADER.parent), str(c), "-o", str(exe)],
                       check=True, capture_output=True)
        out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return [int(x) for x in out.split()]


@pytest.mark.parametrize("cls,cname", [(_lib.CbRows, "cb_rows"), (_lib.CbPlanDesc, "cb_plan_desc"),
                                       (_lib.CbRequest, "cb_request"), (_lib.CbSpan, "cb_span"),
                                       (_lib.CbPlanInfo, "cb_plan_info")])
def test_struct_layouts_match_the_c_compiler(cls, cname):
    fields = [name for name, _ in cls._fields_]
    size, *offsets = _c_layout(cname, fields)
    assert ctypes.sizeof(cls) == size
    assert [getattr(cls, f).offset for f in fields] == offsets


def test_host_validation_errors_without_a_device(lib):
    rows = _lib.CbRows()
    rc = lib.cb_copy_rows(None, ctypes.byref(rows), 1, 1, 128, _lib.CB_DTYPE_BF16, None, None)
    assert rc == _lib.CB_EINVAL and b"null" in lib.cb_last_error()
    rc = lib.cb_copy_rows(ctypes.byref(rows), ctypes.byref(rows), 1, 1, 128, 7, None, None)
    assert rc == _lib.CB_EINVAL and b"dtype" in lib.cb_last_error()
    rc = lib.cb_copy_rows(ctypes.byref(rows), ctypes.byref(rows), 1, 1, 12, _lib.CB_DTYPE_BF16,
                          None, None)
    assert rc == _lib.CB_EINVAL and b"16" in lib.cb_last_error()
    with pytest.raises(ValueError, match="null"):
        _lib.check(lib.cb_map_install(None, None, None))
    with pytest.raises(ValueError, match="null"):
        _lib.check(lib.cb_map_install_batch(None, None, None, None, 0, None, 0, None))
    total = ctypes.c_int64(0)
    assert lib.cb_batch_workspace_bytes(None, None, 0, ctypes.byref(total)) == _lib.CB_EINVAL
    assert lib.cb_plan_create(None, None) == _lib.CB_EINVAL
    info = _lib.CbPlanInfo()
    assert lib.cb_plan_get_info(None, ctypes.byref(info)) == _lib.CB_EINVAL
    lib.cb_plan_destroy(None)  # a no-op, as free(NULL)
