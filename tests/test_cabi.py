"""The C-ABI library loads without a GPU and exports exactly what
include/oscar_amd.h declares, with the argument types the ctypes binding
uses.  Only the two pure-host size queries are called here."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from oscar_amd import integration
from oscar_amd.kernels import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "oscar_amd.h"

C_TO_CTYPES = {
    "int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t,
    "float": ctypes.c_float, "int": ctypes.c_int32, "oscar_stream_t": ctypes.c_void_p,
}


def declarations():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    decls = {}
    for ret, name, params in re.findall(r"\b(size_t|int)\s+(oscar_\w+)\s*\(([^)]*)\)\s*;", text):
        args = []
        for p in (x.strip() for x in params.split(",") if x.strip()):
            if "*" in p:
                args.append(ctypes.c_void_p)
            else:
                ctype = re.sub(r"\s+\w+$", "", p).replace("const", "").strip()
                args.append(C_TO_CTYPES[ctype])
        decls[name] = (C_TO_CTYPES[ret], args)
    return decls


def test_header_declares_every_bound_symbol_with_matching_types():
    decls = declarations()
    assert len(decls) >= 8
    assert set(decls) == set(_lib.SIGNATURES)
    for name, (res, args) in decls.items():
        bres, bargs = _lib.SIGNATURES[name]
        assert res == bres, name
        assert args == bargs, f"{name}: header {args} vs binding {bargs}"


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built (run __graft_entry__.build())")
    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in declarations():
        assert name in exported, name
        assert getattr(lib, name) is not None


def test_size_queries(lib):
    assert lib.oscar_rotation_operand_bytes(256) == 524288
    assert lib.oscar_rotation_operand_bytes(128) == 0
    assert lib.oscar_paged_decode_workspace_bytes(0, 1, 6, 4, 100, 0) == 0
    assert lib.oscar_paged_decode_workspace_bytes(1, 2, 5, 4, 100, 0) == 0     # Hq % Hk
    assert lib.oscar_paged_decode_workspace_bytes(1, 1, 6, 4, 100, 257) == 0   # tiles per split cap
    for args in [(1, 1, 6, 4, 24579, 0), (8, 1, 6, 4, 6000, 0), (3, 2, 12, 16, 131072, 0),
                 (1, 1, 6, 1, 0, 0), (64, 4, 32, 16, 1 << 20, 0), (2, 1, 6, 4, 24579, 4),
                 (300, 1, 6, 4, 4096, 0), (129, 2, 12, 2, 100, 8)]:
        want = integration.decode_workspace_bytes(*args[:5], tiles_per_split=args[5])
        assert lib.oscar_paged_decode_workspace_bytes(*args) == want, args


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(_lib.OscarKernelError, match="missing"):
        _lib.load()


def test_struct_layouts_match_the_header(tmp_path):
    """The ctypes mirrors of the argument structs have the C compiler's field
    offsets and sizes (a header compiled by gcc against its own declaration)."""
    from oscar_amd.kernels import step

    structs = {"oscar_mtp_layer": step.MtpLayerArgs, "oscar_mtp_step": step.MtpStepArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "oscar_amd.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", str(HEADER.parent), str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                              text=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(got[f"{cname} sizeof"]) == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert int(got[f"{cname} {field}"]) == getattr(cls, field).offset, (cname, field)
    # the mirrors name every field the header declares, in its order
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for cname, cls in structs.items():
        body = re.search(r"typedef struct " + cname + r" \{(.*?)\} " + cname + ";", text, flags=re.S).group(1)
        names = []
        for decl in body.split(";"):
            decl = decl.strip()
            if decl:
                names += [re.sub(r"^.*[\s*]", "", part.strip()) for part in decl.split(",")]
        assert names == [f for f, _ in cls._fields_], cname


def test_noalloc_scratch_size_is_budgeted(tmp_path):
    """The no-allocation decode's device array (resident on every GPU that
    loads the library) is the size the memory plan reserves per device."""
    from oscar_amd import integration

    src = tmp_path / "scratch.c"
    src.write_text('#include <stdio.h>\n#include "oscar_amd.h"\n'
                   'int main(void) { printf("%zu\\n", OSCAR_DECODE_NOALLOC_SCRATCH_BYTES); return 0; }\n')
    exe = tmp_path / "scratch"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", str(HEADER.parent), str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    size = int(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)
    assert size == integration.NOALLOC_SCRATCH_BYTES == 32 << 20
    plan = integration.plan_capacity(integration.MI355X_HBM_BYTES - 20 * 10 ** 9, layers=16)
    bare = (16 * integration.fixed_bytes_per_layer(256, 1, 128, 128, 256, 8192, True)
            + integration.decode_workspace_bytes(256, 1, 6, 4, 262144))
    assert plan["fixed"] == bare + size
