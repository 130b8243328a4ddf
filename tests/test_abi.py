"""The C-ABI library loads without a GPU and exports every function that
include/ic_abi.h declares (no compute calls here)."""

import ctypes
import os

import pytest

from int_crush_converter_amd import _native as nat


@pytest.fixture(scope="module")
def libicq():
    if not os.path.exists(nat.LIB_PATH):
        from int_crush_converter_amd import build
        build.build()
    return ctypes.CDLL(nat.LIB_PATH)


def test_header_declares_functions():
    names = nat.header_functions()
    assert "ic_rotate_rows" in names and "ic_last_error" in names
    assert len(names) >= 10


def test_library_exports_header_symbols(libicq):
    missing = [n for n in nat.header_functions() if not hasattr(libicq, n)]
    assert not missing, f"symbols declared in ic_abi.h but not exported: {missing}"


def test_loader_signatures_cover_header():
    assert set(nat.header_functions()) <= set(nat._SIGS), "every ABI function needs a ctypes signature"


def test_version_and_error_without_gpu(libicq):
    libicq.ic_abi_version.restype = ctypes.c_int
    assert libicq.ic_abi_version() == 1
    libicq.ic_last_error.restype = ctypes.c_char_p
    assert isinstance(libicq.ic_last_error(), bytes)


def test_argument_validation_without_gpu(libicq):
    """Bad arguments are rejected on the host before any HIP call."""
    nat.load(require_gpu=False)
    L = nat._lib
    rc = L.ic_rotate_rows(None, 0, 4, 16, 16, None, 16, 16, 16, 0.0, None, None)
    assert rc == -1 and b"null" in L.ic_last_error()
    rc = L.ic_rotate_rows(1, 0, 4, 16, 16, 1, 16, 16, 12, 0.0, None, None)
    assert rc == -1 and b"power of 2" in L.ic_last_error()


# ------------------------------------------------ signatures: header, loader, stubs

def _header_sigs() -> dict[str, tuple[str, list[str]]]:
    """name -> (return kind, [argument kinds]) parsed from include/ic_abi.h."""
    import re
    with open(nat.HEADER_PATH) as f:
        text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    text = re.sub(r"#.*", "", text)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(ic_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        args = [] if params in ("", "void") else [_c_kind(p) for p in params.split(",")]
        out[name] = (_c_kind(ret + " x"), args)
    return out


def _c_kind(decl: str) -> str:
    d = " ".join(decl.split())
    if "*" in d:
        return "ptr"
    t = d.rsplit(" ", 1)[0].replace("const ", "")
    return {"int": "i32", "int64_t": "i64", "float": "f32", "double": "f64", "unsigned long long": "u64",
            "void": "void"}[t]


def _ctypes_kind(t) -> str:
    if t in (ctypes.c_void_p, ctypes.c_char_p) or (isinstance(t, type) and issubclass(t, ctypes._Pointer)):
        return "ptr"
    return {ctypes.c_int: "i32", ctypes.c_int64: "i64", ctypes.c_float: "f32", ctypes.c_double: "f64",
            ctypes.c_ulonglong: "u64"}[t]


def test_loader_signatures_match_header():
    """Every ctypes signature in _native has the header's argument count and
    kinds (pointer / int32 / int64 / float) and return kind."""
    hdr = _header_sigs()
    assert set(hdr) == set(nat.header_functions())
    for name, (ret, args) in hdr.items():
        res, argtypes = nat._SIGS[name]
        got = [_ctypes_kind(a) for a in argtypes]
        assert got == args, (name, got, args)
        assert _ctypes_kind(res) == ret, (name, res, ret)


def test_integration_stubs_match_header():
    """The ctypes bindings shown in INTEGRATION.md (the reference-side
    stubs) agree with include/ic_abi.h argument by argument."""
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with open(os.path.join(root, "INTEGRATION.md")) as f:
        md = f.read()
    code = "\n".join(re.findall(r"```python\n(.*?)```", md, flags=re.S))
    alias = {"_P": "ptr", "_I": "i32", "_L": "i64", "_F": "f32", "ctypes.c_ulonglong": "u64",
             "ctypes.c_char_p": "ptr"}

    def kinds(lst: str) -> list[str]:
        items = [x.strip() for x in re.split(r",(?![^(]*\))", lst) if x.strip()]
        return ["ptr" if x.startswith("ctypes.POINTER") else alias[x] for x in items]

    hdr = _header_sigs()
    bound = {}
    for m in re.finditer(r'"(ic_[a-z0-9_]+)":\s*\(\[([^\]]*)\],\s*([\w\.]+)\)', code):
        bound[m.group(1)] = (kinds(m.group(2)), alias[m.group(3)])
    for m in re.finditer(r"\.(ic_[a-z0-9_]+)\.argtypes\s*=\s*\[([^\]]*)\]", code):
        bound[m.group(1)] = (kinds(m.group(2)), None)
    assert len(bound) >= 10, sorted(bound)
    for name, (args, ret) in bound.items():
        assert name in hdr, name
        assert args == hdr[name][1], (name, args, hdr[name][1])
        if ret is not None:
            assert ret == hdr[name][0], (name, ret, hdr[name][0])


def test_host_tensor_refused_before_the_call(libicq):
    """A tensor in host memory never reaches the library: the loader's
    wrapper raises ValueError before calling (no GPU needed); a NULL is
    refused by the library's own checks."""
    import torch
    nat.load(require_gpu=False)
    L = nat._lib
    x = torch.zeros(4, 16)
    with pytest.raises(ValueError, match="cpu tensor"):
        L.ic_rotate_rows_exact(x, 0, 4, 16, 16, x, 16, 16, 16, 0.0, None, None)
    with pytest.raises(ValueError, match="cpu tensor"):
        L.ic_hessian_inverse(torch.eye(4), 1, 4, 0.01, 0, None, None, None)
    rc = L.ic_rotate_hessian_exact(None, None, 1, 16, 16, 16, 0, None)
    assert rc == -1 and b"null" in L.ic_last_error()
    rc = L.ic_greedy(1, 1, 1, 2, 1, 4, 4, 1, 4, 1, None)
    assert rc == -1 and b"scale_kind" in L.ic_last_error()


def test_every_entry_point_checks_its_arguments_without_gpu(libicq):
    """Each entry point called with NULL for every pointer and small sizes
    answers on the host: a status entry point returns -1 with a message
    (before any GPU work), a size query returns a count.  Run under the
    host-sanitizer build (asan_check.py) this walks every argument check."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("NULL-argument calls are for a host without a GPU")
    nat.load(require_gpu=False)
    raw = ctypes.CDLL(nat.LIB_PATH)
    values = {"ptr": None, "i32": 1, "i64": 16, "f32": 0.5, "f64": 0.5, "u64": 1}
    ctype = {"ptr": ctypes.c_void_p, "i32": ctypes.c_int, "i64": ctypes.c_int64, "f32": ctypes.c_float,
             "f64": ctypes.c_double, "u64": ctypes.c_ulonglong}
    raw.ic_last_error.restype = ctypes.c_char_p
    checked = 0
    for name, (ret, args) in _header_sigs().items():
        if name in ("ic_abi_version", "ic_last_error") or not args:
            continue
        fn = getattr(raw, name)
        fn.argtypes = [ctype[a] for a in args]
        fn.restype = ctype[ret] if ret != "void" else None
        rc = fn(*[values[a] for a in args])
        if ret == "i32" and "ptr" in args:
            assert rc == -1, (name, rc)
            assert raw.ic_last_error(), name
            checked += 1
        elif ret == "i64":
            assert rc >= 0, (name, rc)
    assert checked >= 20
