"""The C-ABI libraries load and export every function their headers declare
(CPU: no kernel is launched), and the ctypes signature table agrees with the
header's parameter lists."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from mantisnet import _hip_api, _native

INCLUDE = Path(__file__).resolve().parents[1] / "include"


def _declarations(header: str) -> dict[str, int]:
    """Function name -> parameter count for every prototype in the header."""
    text = (INCLUDE / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"\b(?:int32_t|int64_t|void)\s+(\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.mark.parametrize("header,lib", [("hexo_encoder.h", _native.ENCODER_LIB), ("mantis_hip.h", _native.HIP_LIB)])
def test_library_exports_every_declared_symbol(header, lib):
    decls = _declarations(header)
    assert len(decls) >= 9, decls
    so = ctypes.CDLL(str(lib))
    missing = [name for name in decls if not hasattr(so, name)]
    assert not missing, missing


def test_ctypes_signatures_match_header():
    decls = _declarations("mantis_hip.h")
    assert set(_hip_api.SIGNATURES) == set(decls)
    for name, (args, _res) in _hip_api.SIGNATURES.items():
        assert len(args) == decls[name], name


def test_substage_struct_matches_header():
    text = (INCLUDE / "mantis_hip.h").read_text()
    body = re.search(r"typedef struct mantis_substage \{(.*?)\} mantis_substage;", text, flags=re.S).group(1)
    fields = re.findall(r"(\w+);", body)
    assert fields == [name for name, _ in _hip_api.MantisSubstage._fields_]
    # every field is a pointer or an int64: 8 bytes each, no padding
    assert ctypes.sizeof(_hip_api.MantisSubstage) == 8 * len(fields)


def test_versions_answer_without_a_gpu():
    assert _native.encoder().hexo_repr_version() == 9
    assert _native.hip().mantis_hip_version() > 0


def test_every_ops_call_passes_the_declared_argument_count():
    # each `_lib().mantis_*(...)` call in the ops layer against the header's
    # parameter list (ctypes would only notice a wrong count at run time)
    src = (Path(__file__).resolve().parents[1] / "hexo-shrimp-bot_amd" / "mantisnet" / "ops.py").read_text()
    decls = _declarations("mantis_hip.h")
    seen = 0
    for m in re.finditer(r"_lib\(\)\.(mantis_\w+)\(", src):
        name, k, depth, n, last = m.group(1), m.end(), 1, 1, ""
        while depth:
            ch = src[k]
            if ch in "([":
                depth += 1
            elif ch in ")]":
                depth -= 1
            elif ch == "," and depth == 1:
                n += 1
            if not ch.isspace() and depth:
                last = ch
            k += 1
        if last == ",":
            n -= 1
        assert n == decls[name], (name, n, decls[name])
        seen += 1
    assert seen >= 20


def test_noalloc_size_guard_holds_at_int64_scale_counts():
    # the workspace size and the no-allocation entry point's guard with counts
    # whose byte products would overflow int64: the guard answers
    # MANTIS_E_SIZE before any device call (none is made: the pointers are
    # never dereferenced, so stand-in addresses serve), and the size query -1
    hip = _native.hip()
    assert hip.mantis_stable_key_order_workspace(10, 3) == 16 + 80
    for n_entries, n_keys in ((0, 2 ** 62), (2 ** 61, 1), (2 ** 63 - 1, 2 ** 63 - 1), (2 ** 60 + 1, 2 ** 61)):
        assert hip.mantis_stable_key_order_workspace(n_entries, n_keys) == -1
    fake = ctypes.c_void_p(0x1000)
    limit = 40 << 20
    for n_entries, n_keys in ((0, 2 ** 62), (2 ** 61, 1), (2 ** 63 - 1, 2 ** 63 - 1), (limit // 8 + 1, 1),
                              (0, limit // 4 + 1)):
        rc = hip.mantis_stable_key_order_noalloc(fake, fake, fake, n_entries, n_keys, fake, fake, fake, None, None)
        assert rc == 3, (n_entries, n_keys, rc)
