"""The C-ABI library loads and exports every entry point include/trida_hip.h declares (no GPU needed,
no compute calls)."""
import ctypes
import re
from pathlib import Path

import pytest

from trida_stack_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "trida_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(trida_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "trida_greedy_accept" in names and "trida_version" in names


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libtrida_hip.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(declared_functions()) <= set(_lib.SIGNATURES), set(declared_functions()) - set(_lib.SIGNATURES)


def test_host_only_entry_points():
    lib = _lib.load()
    assert lib.trida_version() >= 100
    n = lib.trida_greedy_accept_scratch_bytes(1, 33, 151936, 0, 0)
    assert n > 0
    # argument validation happens before any launch: R < K + 1 is rejected with TRIDA_ERR_ARG
    rc = lib.trida_greedy_accept(1, 0, 1, 4, 10, 40, 10, 1, 4, 4, None, None, None, 1, 1, 1, 1, n, 0, None)
    assert rc == _lib.TRIDA_ERR_ARG
    assert b"R >= K + 1" in lib.trida_last_error()


def test_mode_registry_matches_reference_launcher():
    """The --mode values of the reference launcher (inference/zoro-1/serve.py:55-58)."""
    from trida_stack_amd.engine import MODES
    from trida_stack_amd import cli

    assert set(MODES) == {"causal", "self-spec"}
    import pytest as _p
    with _p.raises(SystemExit):
        cli.main(["--mode", "decide"])
