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


_C_TO_FFM = {"int": "I32", "int32_t": "I32", "int64_t": "I64", "uint64_t": "I64", "float": "F32"}


def header_signatures():
    """export -> [return, *args] as FFM layout names, from the header."""
    text = open(os.path.join(ROOT, "include", "rstr_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"^\s*(int|int64_t|const char\*)\s+(rstr_\w+)\s*\(([^)]*)\);", text,
                                      flags=re.M):
        lay = ["PTR" if "*" in ret else _C_TO_FFM[ret]]
        args = " ".join(args.split())
        if args not in ("", "void"):
            for a in args.split(","):
                a = a.strip()
                lay.append("PTR" if "*" in a else _C_TO_FFM[a.replace("const ", "").split()[0]])
        out[name] = lay
    return out


def test_ffm_binding_table_matches_the_header():
    """The Panama FFM downcall table of the integration notes covers every
    export with the header's argument and return layouts."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = doc[doc.index("(def ^:private signatures"):]
    block = block[:block.index("})")]
    table = {name: lay.split() for name, lay in re.findall(r'"(rstr_\w+)"\s*\[([^\]]*)\]', block)}
    want = header_signatures()
    assert set(table) == set(want), set(table) ^ set(want)
    for name, lay in want.items():
        assert table[name] == lay, (name, table[name], lay)


def test_open_without_device_fails_with_a_message():
    import torch  # noqa: F401  (image check only: no device in this container)
    if torch.cuda.is_available():
        return
    s = ctypes.c_void_p()
    rc = hip.lib().rstr_session_open(0, ctypes.byref(s))
    assert rc != 0
    assert hip.lib().rstr_open_error().decode()
