"""The C-ABI library builds, loads without a GPU and exports every entry point
declared in include/rstr_hip.h (no compute calls here)."""
from __future__ import annotations

import ctypes
import os
import re

from rstr import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "rstr_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(rstr_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_binding_surface():
    syms = declared_symbols()
    assert set(syms) == set(hip.EXPORTS), set(syms) ^ set(hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(hip.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_open_without_device_fails_with_a_message():
    import torch  # noqa: F401  (image check only: no device in this container)
    if torch.cuda.is_available():
        return
    s = ctypes.c_void_p()
    rc = hip.lib().rstr_session_open(0, ctypes.byref(s))
    assert rc != 0
    assert hip.lib().rstr_open_error().decode()
