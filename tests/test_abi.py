"""The C-ABI library loads and exports every symbol include/*.h declares;
host-side argument checks and error mapping work without a GPU."""
import ctypes
import glob
import os
import re

import pytest

import channel_amd as ca

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(chn_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "chn_gemv_q4" in names and "chn_init" in names
    assert len(names) >= 10


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(ca.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_every_declared_symbol():
    missing = [n for n in declared_functions() if n not in ca.PROTOTYPES]
    assert not missing, missing
    extra = [n for n in ca.PROTOTYPES if n not in declared_functions()]
    assert not extra, extra


def test_no_oracle_in_product():
    """The product library and package never reference the oracle."""
    for path in glob.glob(os.path.join(ROOT, "channel_amd", "**", "*.*"), recursive=True):
        if path.endswith((".py", ".hip", ".h", ".cpp")):
            src = open(path).read()
            assert "oracle" not in src.replace("oracles", ""), path
    data = open(ca.LIB_PATH, "rb").read()
    assert b"orc_" not in data


def test_null_context_and_bad_args_are_rejected():
    lib = ca.lib
    assert lib.chn_gemv_q4(None, None, None, None, 1, 32) == -1
    assert lib.chn_alloc(None, 16, None) == -1
    assert lib.chn_init(0, None) == -1


@pytest.mark.skipif(ca.device_count() > 0, reason="a HIP device is visible")
def test_init_without_device_reports_no_device():
    with pytest.raises(ca.ChannelError) as e:
        ca.Context(0)
    assert e.value.status == "NoDevice"


def declared_prototypes():
    """name -> list of parameter classes ('ptr', 'u32', 'u64', 'int', 'f32',
    'size') parsed from the header declarations."""
    protos = {}
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for name, params in re.findall(r"\b(chn_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            params = params.strip()
            classes = []
            if params and params != "void":
                for p in params.split(","):
                    p = " ".join(p.split())
                    if "*" in p or "chn_progress_fn" in p:
                        classes.append("ptr")
                    elif p.startswith(("uint32_t", "const uint32_t")):
                        classes.append("u32")
                    elif p.startswith("uint64_t"):
                        classes.append("u64")
                    elif p.startswith("size_t"):
                        classes.append("size")
                    elif p.startswith("float"):
                        classes.append("f32")
                    elif p.startswith("int"):
                        classes.append("int")
                    else:
                        classes.append("?" + p)
            protos[name] = classes
    return protos


def _ctype_class(t):
    if t in (ctypes.c_void_p, ctypes.c_char_p) or (isinstance(t, type) and issubclass(t, ctypes._Pointer)):
        return "ptr"
    return {ctypes.c_uint32: "u32", ctypes.c_uint64: "u64", ctypes.c_size_t: "size", ctypes.c_float: "f32",
            ctypes.c_int: "int"}.get(t, "?" + repr(t))


def test_python_prototypes_match_header_parameters():
    """Every ctypes prototype has the header's parameter count and classes."""
    protos = declared_prototypes()
    assert len(protos) == len(declared_functions())
    bad = []
    same = {"u64": "size"}   # c_uint64 is c_size_t on LP64
    for name, (_, args) in ca.PROTOTYPES.items():
        got = [same.get(c, c) for c in (_ctype_class(a) for a in args)]
        want = [same.get(c, c) for c in protos[name]]
        if got != want:
            bad.append((name, got, want))
    assert not bad, bad
