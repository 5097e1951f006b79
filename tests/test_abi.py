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
