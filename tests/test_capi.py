"""The C-ABI library loads without a GPU, exports every symbol include/anna_mi.h
declares, and rejects bad arguments before launching anything."""

import ctypes
import re
from pathlib import Path

import pytest

from anna_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "anna_mi.h"


def declared_symbols() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(anna_mi_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 6
    for name in names:
        assert hasattr(lib, name), f"{name} declared in anna_mi.h but not exported"


def test_every_declared_symbol_has_a_binding():
    for name in declared_symbols():
        if name in ("anna_mi_last_error", "anna_mi_abi_version", "anna_mi_source_hash"):
            continue
        assert name in _lib.PROTOTYPES or name in _lib.RAW_PROTOTYPES, f"{name} has no ctypes prototype"


def test_decode_args_binding_matches_the_c_struct():
    import ctypes

    assert _lib.load().anna_mi_sizeof_decode_args() == ctypes.sizeof(_lib.DecodeArgs)
    assert _lib.load().anna_mi_sizeof_tq_decode_args() == ctypes.sizeof(_lib.TQDecodeArgs)
    assert _lib.load().anna_mi_sizeof_moe_mlp_args() == ctypes.sizeof(_lib.MoeMlpArgs)
    assert _lib.load().anna_mi_sizeof_tq_append_args() == ctypes.sizeof(_lib.TQAppendArgs)
    assert _lib.load().anna_mi_sizeof_tq_pack_args() == ctypes.sizeof(_lib.TQPackArgs)
    assert _lib.load().anna_mi_sizeof_tq_rows_append_args() == ctypes.sizeof(_lib.TQRowsAppendArgs)


def test_library_is_stamped_with_the_tree_sources():
    from anna_amd import build

    assert _lib.load().anna_mi_source_hash().decode() == build.source_hash()


def test_abi_version_matches_header():
    version = int(re.search(r"#define ANNA_MI_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert _lib.load().anna_mi_abi_version() == version


def test_argument_errors_are_reported_without_launching():
    with pytest.raises(RuntimeError, match="null pointer"):
        _lib.call("anna_mi_int4_linear", None, 0, 1, 8, 8, None, 8, 1, None, 2, None, 1, 128, None, None)
    with pytest.raises(RuntimeError, match="bad dtype"):
        _lib.call("anna_mi_int4_linear", 16, 7, 1, 8, 8, 16, 8, 1, 16, 2, 16, 1, 128, 16, None)
    with pytest.raises(RuntimeError, match="packed columns"):
        _lib.call("anna_mi_int4_linear", 16, 0, 1, 64, 64, 16, 8, 1, 16, 2, 16, 1, 128, 16, None)
