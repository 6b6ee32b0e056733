"""The library-GEMM solution file read at run time (PyTorch TunableOp's results format): validators for the
ROCm / PyTorch build and gfx950, and one entry per projection shape of the batch-64 decode step."""
import csv
import os

from trida_stack_amd import model as M


def test_gemm_choices_file_shapes():
    rows = list(csv.reader(open(M.GEMM_CHOICES)))
    val = {r[1]: r[2] for r in rows if r[0] == "Validator"}
    assert val["GCN_ARCH_NAME"].startswith("gfx950") and "PT_VERSION" in val and "HIPBLASLT_VERSION" in val
    ops = [r for r in rows if r[0] != "Validator"]
    shapes = set()
    for op, sig, sol, ms in ops:
        assert op == "GemmTunableOp_BFloat16_TN" and sol.split("_")[0] in ("Gemm", "Default")
        n, m, k = (int(x) for x in sig.split("_")[1:4])
        assert m == 64 * 33 and float(ms) > 0
        shapes.add((n, k))
    # GDN in, GDN out, gate/up, down, qkv, attention out, LM head of the 4B-shape hybrid
    assert shapes == {(8224, 2560), (2560, 2048), (19456, 2560), (2560, 9728), (10240, 2560), (2560, 4096),
                      (248320, 2560)}


def test_gemm_choices_switch(monkeypatch):
    monkeypatch.setenv("TRIDA_GEMM_CHOICES", "0")
    assert M.use_gemm_choices() is False
    monkeypatch.delenv("TRIDA_GEMM_CHOICES")
    assert M.use_gemm_choices(os.path.join(os.path.dirname(M.GEMM_CHOICES), "no_such_file.csv")) is False
