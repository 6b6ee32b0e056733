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


def test_sampling_argument_checks():
    """The sampled-acceptance entry points reject bad sampling parameters before touching memory
    (dummy non-null pointers; nothing is launched)."""
    lib = _lib.load()
    n = lib.trida_sample_accept_scratch_bytes(64, 33, 248320, 32)
    assert n > 64 * 33 * 20
    P = 256  # a dummy, aligned, non-null address

    def stats(T=0.7, k=0, p=0.95, V=1000):
        return lib.trida_truncate_stats(P, 1, 2, V, 2 * V, V, T, k, p, -1, 0, P, P, P, P, None, None)

    for kw, text in [(dict(T=0.0), b"temperature"), (dict(T=float("inf")), b"temperature"),
                     (dict(p=0.0), b"top_p"), (dict(p=1.5), b"top_p"), (dict(k=-1), b"top_k"),
                     (dict(k=5000, V=10000), b"top_k")]:
        assert stats(**kw) == _lib.TRIDA_ERR_ARG, kw
        assert text in lib.trida_last_error(), (kw, lib.trida_last_error())
    # top_k >= V disables top-k, so it is not an error; K above one wave is
    rc = lib.trida_sample_accept(P, 1, 66, 100, 6600, 100, P, 6500, 100, P, 65, 65, None, P, 65, P, None,
                                 0.7, 0, 0.9, -1, P, P, P, None, P, P, n, None)
    assert rc == _lib.TRIDA_ERR_ARG and b"K <= 64" in lib.trida_last_error()
    rc = lib.trida_sample_accept(P, 1, 33, 100, 3300, 100, P, 3200, 100, P, 32, 32, None, P, 32, P, None,
                                 0.7, 0, 0.9, -1, P, P, P, None, P, P, 16, None)
    assert rc == _lib.TRIDA_ERR_WORKSPACE


def test_mode_registry_matches_reference_launcher():
    """The --mode values of the reference launcher (inference/zoro-1/serve.py:55-58), plus "diffusion",
    the vLLM plugin's pure block-diffusion decode (qwen3_5_diffusion.py:1180-1270)."""
    from trida_stack_amd.engine import MODES
    from trida_stack_amd import cli

    assert {"causal", "self-spec"} <= set(MODES) and set(MODES) - {"causal", "self-spec"} == {"diffusion"}
    import pytest as _p
    with _p.raises(SystemExit):
        cli.main(["--mode", "decide"])


def declared_param_counts():
    """name -> number of parameters of each declaration in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(trida_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_binding_arity_matches_header():
    """Every ctypes signature has exactly the header's parameter count (a miscount would shift every
    argument after it)."""
    counts = declared_param_counts()
    assert counts, "no declarations parsed"
    bad = {n: (counts[n], len(_lib.SIGNATURES[n][1])) for n in counts if counts[n] != len(_lib.SIGNATURES[n][1])}
    assert not bad, bad


def test_gdr_chunk_argument_checks():
    """The chunked GDR entry point rejects bad shapes and modes before launching (dummy pointers)."""
    lib = _lib.load()
    P = 256
    assert lib.trida_gdr_chunk_workspace_bytes(1, 64, 16) == 0
    # per (chunk, head): the larger of the general path's T hi / lo + M (3 x 64 x 64 bf16) and the prefix
    # kernels' T and M fragments and decays (19456 bytes)
    assert lib.trida_gdr_chunk_workspace_bytes(1, 4096, 16) == 64 * 16 * max(3 * 64 * 64 * 2, 19456)

    def call(T=100, Dk=128, Dv=128, mode=1, ws=None, ws_bytes=0, n_keep=None):
        return lib.trida_gdr_chunk(P, P, P, P, P, P, P, P, n_keep, 1, 1, T, 16, 16, Dk, Dv, mode, 0, 0.1, ws,
                                   ws_bytes, None, None, None)

    assert call(Dk=256) == _lib.TRIDA_ERR_ARG and b"Dk" in lib.trida_last_error()
    assert call(Dv=24) == _lib.TRIDA_ERR_ARG
    assert call(mode=2) == _lib.TRIDA_ERR_ARG and b"causal_mode 2" in lib.trida_last_error()
    assert call(T=64, mode=2, n_keep=P) == _lib.TRIDA_ERR_ARG
    assert call(T=100) == _lib.TRIDA_ERR_WORKSPACE


def test_ws_fragment_order_host_checks():
    """The fragment order of the weight-streaming GEMM's X: its size and the argument checks of the entry
    points that read or write it (dummy pointers; nothing is launched)."""
    lib = _lib.load()
    assert lib.trida_ws_frag_elems(2560) == 2560 // 32 * 3 * 64 * 8
    assert lib.trida_ws_frag_elems(100) == 0
    P = 256
    # partial planes have no fragment order; unknown flag bits; M above 48
    assert lib.trida_wsgemm_ex(P, 0, None, 1e-6, P, 4, 64, 256, 1, P, 0, 2, None) == _lib.TRIDA_ERR_ARG
    assert lib.trida_wsgemm_ex(P, 0, None, 1e-6, P, 4, 64, 256, 0, P, 0, 4, None) == _lib.TRIDA_ERR_ARG
    assert lib.trida_wsgemm_ex(P, 0, None, 1e-6, P, 49, 64, 256, 0, P, 0, 1, None) == _lib.TRIDA_ERR_ARG
    # the RMSNorm prologue takes no partial planes
    assert lib.trida_wsgemm_ex(P, 256, P, 1e-6, P, 4, 64, 256, 1, P, 0, 0, None) == _lib.TRIDA_ERR_ARG
    assert lib.trida_ws_frag(P, 256, 49, 256, P, None) == _lib.TRIDA_ERR_ARG
    assert lib.trida_residual_parts_frag(P, 256, None, 0, 0, 49, 256, P, P, None) == _lib.TRIDA_ERR_ARG
    assert lib.trida_gated_rmsnorm_frag(P, P, P, P, 49, 2, 128, 256, 1e-6, None) == _lib.TRIDA_ERR_ARG


def test_ws_fragment_offsets_are_a_bijection():
    """The fragment order's element offset (restated from the header's formula) maps the rows < 48 x K
    elements one to one onto [0, trida_ws_frag_elems(K)), and keeps each lane's 8 elements of a k-step
    consecutive (what makes one 16-byte load per lane)."""
    import numpy as np

    K = 96
    m, k = np.meshgrid(np.arange(48), np.arange(K), indexing="ij")
    off = (((k // 32) * 3 + m // 16) * 64 + ((k % 32) // 8) * 16 + m % 16) * 8 + k % 8
    assert np.array_equal(np.sort(off.ravel()), np.arange(_lib.load().trida_ws_frag_elems(K)))
    assert np.all(np.diff(off.reshape(48, K // 8, 8), axis=2) == 1)
