"""The library-GEMM solution file read at run time (PyTorch TunableOp's results format): validators for the
ROCm / PyTorch build and gfx950, and one entry per projection shape of the batch-64 decode step."""
import csv
import os

import pytest

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


@pytest.mark.gpu
def test_runtime_leaves_tunableop_state_alone(gpu, tmp_path):
    """The runtime turns TunableOp lookup on only around its own library GEMMs: a host's settings (off, or
    on with tuning) are what they were before the runtime was built and after its GEMMs ran."""
    import torch

    from trida_stack_amd.model import HybridConfig, TridaRuntime, init_weights

    t = torch.cuda.tunable
    t.set_filename(str(tmp_path / "tunableop_results.csv"))  # anything TunableOp writes stays out of the tree
    cfg = HybridConfig.tiny(vocab=512)
    for state in ((False, False), (True, False), (True, True)):
        t.enable(state[0])
        t.tuning_enable(state[1])
        rt = TridaRuntime(cfg, init_weights(cfg, seed=0), device=gpu)
        c = rt.make_cache(2, max_len=128)
        rt.forward(torch.zeros(2, 60, dtype=torch.long, device=gpu), c, "causal")  # library GEMMs
        torch.cuda.synchronize()
        assert (t.is_enabled(), t.tuning_is_enabled()) == state
    t.tuning_enable(False)
    t.enable(False)
