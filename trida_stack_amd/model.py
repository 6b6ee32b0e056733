"""Hybrid Qwen3.5-style decoder (gated-delta + full attention) on MI355X, with the forwards the
self-speculative decoder needs.

Mirrors the reference runtime API of inference/zoro-1/mlx/trida_mlx/model.py:
  make_cache() / prefill(cache, tokens) / ar_step(cache, tok) / canvas(cache, tokens, n_clean, rows)
  / commit(cache, adv)                                                          (model.py:245-507)
plus draft(cache, tokens), the block-diffusion denoising pass (MASK rows see the whole block).

Every hot op runs in a gfx950 kernel of libtrida_hip.so (attention, GDN conv/prep/recurrence/readout,
rollback, norms, SwiGLU, acceptance); the projections, MLP and LM head are torch GEMMs (hipBLASLt).
Caches are batched device tensors: KV [A, B, Hkv, Lmax, D] bf16, GDN state [L, B, Hv, Dv, Dk] fp32 and
conv window [L, B, Kc-1, C] bf16 (A / L = number of attention / GDN layers). Per-sequence lengths and
RoPE positions live on the device, so every forward of a given (B, T, mode) has fixed launch shapes
and can be captured in a HIP graph.

Forward modes (reference semantics):
  causal  token-causal rows, state persisted (prefill / AR step)
  verify  token-causal rows, nothing persisted; commit(adv) keeps the first adv rows
  canvas  rows < n_clean token-causal, later rows see the whole block (attention) and read the
          block-end GDN state (causal_mode 2, num_clean)                        (model.py:461-484)
  draft   the denoising pass: every row sees the whole block in attention, GDN rows >= 1 read the
          block-end state (causal_mode 2, num_clean 1)
"""
from __future__ import annotations

import json
import math
import os
from dataclasses import asdict, dataclass, field
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from . import kernels as K

DEFAULT_MASK_ID = 248077


@dataclass
class HybridConfig:
    hidden: int = 2560
    n_layers: int = 32
    full_attention_interval: int = 4     # layer i is full attention when (i + 1) % interval == 0
    intermediate: int = 9728
    vocab: int = 248320
    lin_k_heads: int = 16
    lin_v_heads: int = 16
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_kernel: int = 4
    n_heads: int = 16
    n_kv_heads: int = 4
    head_dim: int = 256
    rotary_frac: float = 0.25
    rope_theta: float = 1.0e7
    rms_eps: float = 1e-6
    mask_id: int = DEFAULT_MASK_ID
    tie_embeddings: bool = True
    # per-layer "linear_attention" / "full_attention" (a checkpoint's config.json layer_types); when
    # None, layer i is full attention iff (i + 1) % full_attention_interval == 0
    layer_types: Optional[Tuple[str, ...]] = None

    @property
    def conv_dim(self) -> int:
        return 2 * self.lin_k_heads * self.lin_k_dim + self.lin_v_heads * self.lin_v_dim

    @property
    def value_dim(self) -> int:
        return self.lin_v_heads * self.lin_v_dim

    @property
    def rot_dim(self) -> int:
        return int(self.head_dim * self.rotary_frac)

    def is_attention(self, i: int) -> bool:
        if self.layer_types is not None:
            return self.layer_types[i] == "full_attention"
        return (i + 1) % self.full_attention_interval == 0

    @classmethod
    def four_b(cls) -> "HybridConfig":
        """The 4B-shape hybrid of the end-to-end benchmark: hidden 2560, 32 layers (24 GDN + 8 attention),
        GDN 16 key / 16 value heads of 128, attention 16 q / 4 kv heads of 256, FFN 9728, vocab 248320."""
        return cls()

    @classmethod
    def tiny(cls, vocab: int = 300) -> "HybridConfig":
        """A small configuration for tests (kernel-supported head sizes)."""
        return cls(hidden=128, n_layers=8, intermediate=256, vocab=vocab, lin_k_heads=2, lin_v_heads=4,
                   lin_k_dim=32, lin_v_dim=64, n_heads=4, n_kv_heads=2, head_dim=64, rope_theta=10000.0,
                   mask_id=vocab - 1)

    def n_params(self) -> int:
        h, I = self.hidden, self.intermediate
        gdn = h * (self.conv_dim + self.value_dim + 2 * self.lin_v_heads) + self.value_dim * h
        attn = h * (2 * self.n_heads + 2 * self.n_kv_heads) * self.head_dim + self.n_heads * self.head_dim * h
        mlp = 3 * h * I
        n_attn = sum(self.is_attention(i) for i in range(self.n_layers))
        return self.vocab * h + (self.n_layers - n_attn) * gdn + n_attn * attn + self.n_layers * mlp


def init_weights(cfg: HybridConfig, seed: int = 0, device="cpu", dtype=torch.bfloat16,
                 embed_scale: float = 1.0) -> Dict[str, torch.Tensor]:
    """Random weights of the hybrid architecture (normal(0, 0.02) projections, zero-centred norms at 0,
    gated norm at 1, A_log = log U(1, 16), dt_bias = 1), in the [out, in] layout of torch Linear.
    embed_scale sharpens the tied embedding (tests use it to give greedy decoding structure)."""
    g = torch.Generator(device=device).manual_seed(seed)
    h, I = cfg.hidden, cfg.intermediate

    def nrm(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(dtype)

    w: Dict[str, torch.Tensor] = {"embed": (nrm(cfg.vocab, h).float() * embed_scale).to(dtype),
                                  "final_norm": torch.zeros(h, device=device, dtype=dtype)}
    for i in range(cfg.n_layers):
        p = f"l{i}."
        w[p + "in_norm"] = torch.zeros(h, device=device, dtype=dtype)
        w[p + "post_norm"] = torch.zeros(h, device=device, dtype=dtype)
        w[p + "w_gu"] = nrm(2 * I, h)
        w[p + "w_down"] = nrm(h, I)
        if cfg.is_attention(i):
            w[p + "w_qkv"] = nrm((2 * cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim, h)
            w[p + "q_norm"] = torch.zeros(cfg.head_dim, device=device, dtype=dtype)
            w[p + "k_norm"] = torch.zeros(cfg.head_dim, device=device, dtype=dtype)
            w[p + "w_o"] = nrm(h, cfg.n_heads * cfg.head_dim)
        else:
            w[p + "w_in"] = nrm(cfg.conv_dim + cfg.value_dim + 2 * cfg.lin_v_heads, h)
            bound = 1.0 / math.sqrt(cfg.conv_kernel)
            w[p + "conv_w"] = ((torch.rand(cfg.conv_dim, cfg.conv_kernel, generator=g, device=device) * 2 - 1)
                               * bound).to(dtype)
            w[p + "A_log"] = torch.log(torch.rand(cfg.lin_v_heads, generator=g, device=device) * 15 + 1)
            w[p + "dt_bias"] = torch.ones(cfg.lin_v_heads, device=device, dtype=torch.float32)
            w[p + "gnorm"] = torch.ones(cfg.lin_v_dim, device=device, dtype=dtype)
            w[p + "w_out"] = nrm(h, cfg.value_dim)
    return w


@dataclass
class SeqCache:
    """Batched decode state: KV caches, GDN states and conv windows, per-sequence committed length
    and RoPE position on the device, and the committed token ids on the host (what the state
    encodes). `pending` holds the record of a verify/canvas/draft forward until commit."""
    kv_k: torch.Tensor
    kv_v: torch.Tensor
    state: torch.Tensor
    window: torch.Tensor
    length: torch.Tensor         # [B] int32: committed tokens (KV entries)
    pos: torch.Tensor            # [B] int32: RoPE position of the next token
    tokens: List[List[int]] = field(default_factory=list)
    pending: Optional[dict] = None
    # host-side upper bound of the committed length of every sequence (plans attention key splits;
    # exact after prefill / integer commits, conservative after device-side commits until the decode
    # loop settles it)
    ctx_hint: int = 0

    @property
    def B(self) -> int:
        return self.length.shape[0]

    @property
    def Lmax(self) -> int:
        return self.kv_k.shape[3]

    def snapshot(self):
        """Copy of the recurrent state, conv windows and lengths (KV entries are append-only, so the
        length is enough for them) — SeqCache.snapshot of the reference (model.py:184-190)."""
        assert self.pending is None
        st, win = torch.empty_like(self.state), torch.empty_like(self.window)
        K.gdn_snapshot(self.state, st, self.window, win)
        return st, win, self.length.clone(), self.pos.clone(), [list(t) for t in self.tokens]

    def restore(self, snap) -> None:
        st, win, length, pos, tokens = snap
        assert self.pending is None
        K.gdn_snapshot(st, self.state, win, self.window)
        self.length.copy_(length)
        self.pos.copy_(pos)
        self.tokens = [list(t) for t in tokens]


# hipBLASLt's heuristic picks a kernel about twice as slow for M <= 16 rows as for M = 17 at the decode
# projection shapes (gate/up 19456 x 2560: 46.8 us at M = 1..16, 23.5 us at M = 17; gdn in, attention
# qkv / o likewise slower), so the projections of forwards of at most 16 rows (AR steps, canvases of
# 2n - 1 <= 15 rows) run on GEMM_MIN_ROWS rows, the extra rows zero and their outputs unused.
GEMM_MIN_ROWS = 17


class _Scratch:
    """Per-(B, T) activation buffers, reused across forwards (fixed addresses for graph capture). The GEMM
    operands are allocated with Np >= B * T rows (zeros past B * T; see GEMM_MIN_ROWS); the attributes
    without `_p` are the B * T-row views the row-wise kernels use."""

    def __init__(self, cfg: HybridConfig, B: int, T: int, n_gdn: int, dev, ws_parts: int = 0):
        bf = dict(dtype=torch.bfloat16, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        N = B * T
        Np = GEMM_MIN_ROWS if N < GEMM_MIN_ROWS else N
        self.N, self.Np = N, Np
        h = cfg.hidden
        W_in = cfg.conv_dim + cfg.value_dim + 2 * cfg.lin_v_heads
        W_qkv = (2 * cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim
        self.h = torch.empty(N, h, **bf)
        self.x_p = torch.zeros(Np, h, **bf)
        self.r_p = torch.zeros(Np, h, **bf)
        self.gu_p = torch.zeros(Np, 2 * cfg.intermediate, **bf)
        self.act_p = torch.zeros(Np, cfg.intermediate, **bf)
        self.proj_p = torch.zeros(Np, W_in, **bf)
        self.qkv_p = torch.zeros(Np, W_qkv, **bf)
        self.o_att_p = torch.zeros(Np, cfg.n_heads * cfg.head_dim, **bf)
        self.yn_p = torch.zeros(Np, cfg.lin_v_heads * cfg.lin_v_dim, **bf)
        self.x, self.r, self.gu, self.act = self.x_p[:N], self.r_p[:N], self.gu_p[:N], self.act_p[:N]
        self.proj = self.proj_p[:N].view(B, T, W_in)
        self.qkv = self.qkv_p[:N].view(B, T, W_qkv)
        self.o_att = self.o_att_p[:N].view(B, T, cfg.n_heads, cfg.head_dim)
        self.yn = self.yn_p[:N].view(N, cfg.lin_v_heads, cfg.lin_v_dim)
        self.q_att = torch.empty(B, T, cfg.n_heads, cfg.head_dim, **bf)
        self.y = torch.empty(B, T, cfg.lin_v_heads, cfg.lin_v_dim, **bf)
        self.q = torch.empty(B, T, cfg.lin_k_heads, cfg.lin_k_dim, **bf)
        self.win_tmp = torch.empty(B, cfg.conv_kernel - 1, cfg.conv_dim, **bf)
        # per-GDN-layer block rows kept for commit (stacked so one restore launch covers every layer)
        self.k_rec = torch.empty(n_gdn, B, T, cfg.lin_k_heads, cfg.lin_k_dim, **bf)
        self.v_rec = torch.empty(n_gdn, B, T, cfg.lin_v_heads, cfg.lin_v_dim, **bf)
        self.g_rec = torch.empty(n_gdn, B, T, cfg.lin_v_heads, **f32)
        self.b_rec = torch.empty(n_gdn, B, T, cfg.lin_v_heads, **f32)
        self.pre_rec = torch.empty(n_gdn, B, T, cfg.conv_dim, **bf)
        # split-K partial planes of the weight-streaming GEMM ([kg, N, hidden] fp32), when it runs here
        self.parts = torch.empty(max(1, ws_parts) * N * h, **f32) if ws_parts else None
        self.ss = torch.empty(N, (h + 255) // 256, **f32) if ws_parts else None  # per-chunk sums of h^2
        # the fused forward's GEMM inputs in the weight-streaming GEMM's fragment order (h, the SwiGLU
        # output, the gated-norm output), written by their producers
        frag = ws_parts and N <= K.WS_MAX_M
        self.hf = torch.empty(K.ws_frag_numel(h), **bf) if frag else None
        self.actf = torch.empty(K.ws_frag_numel(cfg.intermediate), **bf) if frag else None
        self.ynf = torch.empty(K.ws_frag_numel(cfg.lin_v_heads * cfg.lin_v_dim), **bf) if frag else None
        self.oattf = torch.empty(K.ws_frag_numel(cfg.n_heads * cfg.head_dim), **bf) if frag else None
        # the gated RMSNorm's per-8-column sums of squares of the GDN output, when the recurrence leaves them
        # for the out projection (gdr_recurrent_gnorm)
        self.gss = (torch.empty(N * cfg.lin_v_heads * max(1, cfg.lin_v_dim // 8), **f32)
                    if frag and cfg.lin_v_dim % 32 == 0 else None)


GEMM_CHOICES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_choices_gfx950.csv")


def use_gemm_choices(path: str = GEMM_CHOICES) -> bool:
    """Library GEMM solutions measured per shape of the batch-64 decode step on MI355X (hipBLASLt or rocBLAS,
    whichever ran fastest; PyTorch TunableOp's results format, lookup only, no tuning at run time). Shapes
    the file does not list keep the library's own heuristic; a file written for another library version
    or GPU is ignored by TunableOp's validators. TRIDA_GEMM_CHOICES=0 turns it off.

    Loads the entries into TunableOp's results (process-wide: a host that enables TunableOp for its own
    matmuls of these exact shapes would find them there) without enabling TunableOp; the runtime turns
    the lookup on only around its own library GEMMs (_GemmChoices)."""
    if os.environ.get("TRIDA_GEMM_CHOICES", "1") == "0" or not os.path.exists(path):
        return False
    return bool(torch.cuda.tunable.read_file(path))


class _GemmChoices:
    """TunableOp lookup (no tuning) around one of the runtime's own library GEMMs, the caller's TunableOp
    state restored afterwards: a host application that embeds the runtime keeps its own settings."""

    def __init__(self, on: bool):
        self.on = on

    def __enter__(self):
        if self.on:
            t = torch.cuda.tunable
            self.prev = (t.is_enabled(), t.tuning_is_enabled())
            t.tuning_enable(False)
            t.enable(True)
        return self

    def __exit__(self, *exc):
        if self.on:
            t = torch.cuda.tunable
            t.enable(self.prev[0])
            t.tuning_enable(self.prev[1])
        return False


class TridaRuntime:
    """The self-spec runtime over one model (see the module docstring for the mode semantics)."""

    def __init__(self, cfg: HybridConfig, weights: Dict[str, torch.Tensor], device="cuda:0",
                 prefill_chunk: int = 512, gemm_choices: bool = True):
        """gemm_choices: look the runtime's own library GEMMs up in the bundled solution file
        (use_gemm_choices), with TunableOp switched on only around those calls."""
        self.cfg = cfg
        self.dev = torch.device(device)
        self._choices = _GemmChoices(self.dev.type == "cuda" and gemm_choices and use_gemm_choices())
        self.w = {k: v.to(self.dev) for k, v in weights.items()}
        self.prefill_chunk = prefill_chunk
        self.attn_layers = [i for i in range(cfg.n_layers) if cfg.is_attention(i)]
        self.gdn_layers = [i for i in range(cfg.n_layers) if not cfg.is_attention(i)]
        self._slot = {}
        for j, i in enumerate(self.attn_layers):
            self._slot[i] = j
        for j, i in enumerate(self.gdn_layers):
            self._slot[i] = j
        self._scratch: Dict[tuple, _Scratch] = {}
        self._head_bufs: Dict[tuple, tuple] = {}  # argmax-head split buffers per row count
        self.ws: Dict[str, tuple] = {}
        self.ws_parts = 0
        self.ws_fused = False
        if self.use_wsgemm:
            self._shuffle_weights()
        self.skip_rows = False
        self.mask_id = cfg.mask_id
        self.progress_cb = None  # optional fn(tokens done this call) after each prefill chunk (model.py:241)

    # ---------------------------------------------------------------- cache
    def make_cache(self, batch: int = 1, max_len: int = 4096) -> SeqCache:
        c = self.cfg
        bf = dict(dtype=torch.bfloat16, device=self.dev)
        A, L = len(self.attn_layers), len(self.gdn_layers)
        return SeqCache(
            kv_k=torch.zeros(A, batch, c.n_kv_heads, max_len, c.head_dim, **bf),
            kv_v=torch.zeros(A, batch, c.n_kv_heads, max_len, c.head_dim, **bf),
            state=torch.zeros(L, batch, c.lin_v_heads, c.lin_v_dim, c.lin_k_dim, dtype=torch.float32, device=self.dev),
            window=torch.zeros(L, batch, c.conv_kernel - 1, c.conv_dim, **bf),
            length=torch.zeros(batch, dtype=torch.int32, device=self.dev),
            pos=torch.zeros(batch, dtype=torch.int32, device=self.dev),
            tokens=[[] for _ in range(batch)])

    def grow_cache(self, cache: SeqCache, max_len: int) -> None:
        """Raises the KV capacity of `cache` to max_len positions in place (the committed entries are
        copied; the recurrent state and conv windows do not depend on the capacity)."""
        if max_len <= cache.Lmax:
            return
        A = cache.kv_k.shape[0]
        shape = (A, cache.B, self.cfg.n_kv_heads, max_len, self.cfg.head_dim)
        for name in ("kv_k", "kv_v"):
            old = getattr(cache, name)
            new = torch.zeros(shape, dtype=old.dtype, device=old.device)
            new[:, :, :, : old.shape[3]].copy_(old)
            setattr(cache, name, new)

    def scratch(self, B: int, T: int) -> _Scratch:
        key = (B, T)
        s = self._scratch.get(key)
        if s is None:
            parts = self.ws_parts if B * T <= K.WS_MAX_M else 0
            s = self._scratch[key] = _Scratch(self.cfg, B, T, len(self.gdn_layers), self.dev, ws_parts=parts)
        return s

    # projection -> epilogue of the weight-streaming GEMM: bf16 outputs feed the GDN / attention kernels,
    # the out-projections and the MLP down projection leave fp32 partial planes for add_rmsnorm_parts,
    # gate/up runs with the SwiGLU epilogue
    _WS_ROLE = {"w_in": K.WS_STORE, "w_qkv": K.WS_STORE, "w_out": K.WS_PARTS, "w_o": K.WS_PARTS,
                "w_gu": K.WS_SILU, "w_down": K.WS_PARTS}

    def _shuffle_weights(self) -> None:
        """A second copy of every decoder projection and of the LM head in the weight-streaming layout
        (bf16, the same bytes again: 7.4 + 1.27 GB at the 4B shape), for forwards of <= K.WS_MAX_M rows. A projection whose
        shape the kernel does not take (N % 16, K % 32, or K too long for a whole-K epilogue) keeps the
        hipBLASLt path. When every projection qualifies (and hidden <= 2560), the forward runs fused: the
        RMSNorm in front of a projection moves into its GEMM, with the norm weight folded into the copy's
        columns (bf16(w * (1 + norm)), the Qwen3.5 zero-centred norm)."""
        c = self.cfg
        plans = {}
        for key, wt in self.w.items():
            role = self._WS_ROLE.get(key.split(".", 1)[-1])
            if role is None:
                continue
            N, Kd = wt.shape
            if N % 16 or Kd % 32 or (role == K.WS_SILU and (N // 2) % 8):
                continue
            try:
                plans[key] = (role, K.ws_plan(N, Kd, role))
            except ValueError:
                continue
        proj = [f"l{i}.{k}" for i in range(c.n_layers)
                for k in (("w_qkv", "w_o") if c.is_attention(i) else ("w_in", "w_out")) + ("w_gu", "w_down")]
        self.ws_fused = all(k in plans for k in proj) and K.ss_chunks(c.hidden) <= 10
        for key, (role, kg) in plans.items():
            layer, name = key.split(".", 1)
            norm = None
            if self.ws_fused and name in ("w_in", "w_qkv"):
                norm = self.w[layer + ".in_norm"]
            elif self.ws_fused and name == "w_gu":
                norm = self.w[layer + ".post_norm"]
            wt = self.w[key]
            wp = K.ws_shuffle(wt.contiguous(), pair_halves=role == K.WS_SILU, col_scale=norm)
            self.ws[key] = (wp, wt.shape[0], role, kg)
            if role == K.WS_PARTS:
                self.ws_parts = max(self.ws_parts, kg)
            if name == "w_out" and c.lin_v_dim % 32 == 0:  # the gated-norm fold's projection (ws_gemm_headnorm)
                self.ws_parts = max(self.ws_parts, K.ws_headnorm_planes(wt.shape[0], wt.shape[1], c.lin_v_heads))
        # the LM head (bf16 logits of <= K.WS_MAX_M rows; the fp32 logits_out path keeps hipBLASLt)
        wl = self.w.get("lm_head", self.w.get("embed"))
        if wl is not None and wl.shape[0] % 16 == 0 and wl.shape[1] % 32 == 0:
            try:
                kg = K.ws_plan(wl.shape[0], wl.shape[1], K.WS_STORE)
                self.ws["lm_head"] = (K.ws_shuffle(wl.contiguous()), wl.shape[0], K.WS_STORE, kg)
            except ValueError:
                pass

    # ---------------------------------------------------------------- forward
    # decoder projections of forwards with <= K.WS_MAX_M rows run on the weight-streaming GEMM over
    # pre-shuffled weights (class default; set before building the runtime)
    use_wsgemm = True
    # GDN recurrence form: "chunked" (WY / UT chunks on MFMA, trida_gdr_chunk), "recurrent" (token by
    # token, trida_gdr_recurrent) or "auto" (chunked over more than one chunk of rows, i.e. prefill, and
    # for canvas blocks of large batches, where the single-block MFMA readout wins; recurrent for small
    # batches' blocks and the rollback). Both kernels follow the same recurrence; only "recurrent" makes
    # the rows of a verify block bitwise equal to the same rows decoded one AR step at a time.
    gdr_form = "auto"
    # recurrent blocks of <= 64 rows may run conv + prep + recurrence as one launch
    # (trida_gdn_fused_layer, bit-identical to trida_gdn_prep then trida_gdr_recurrent). Off: each
    # recurrence block would redo its head's q/k front half (16x at batch 1), which measures slower
    # than the separate prep launch (27 vs 23 us per layer at batch 1, 407 vs 236 us at batch 64).
    fused_gdn = False
    # in the fused forward (<= K.WS_MAX_M rows, one staged chunk of recurrence rows), the GDN layer's gated
    # RMSNorm runs inside the recurrence (u = o * w * silu(z) and per-head sums of squares) and the out
    # projection (its per-head rsqrt scale on the partial sums): no gated_rmsnorm launch between them
    fold_gnorm = True
    # fn(i, where, *tensors) or None, for tests that check each layer on its own inputs (never set while a
    # forward is captured into a graph); called in eager forwards with device tensors:
    #   (i, "in", h, r)     the hidden rows [B * T, hidden] (bf16) entering layer i (i = n_layers: the
    #                       final norm) and the previous layer's MLP branch r [B * T, hidden] that h
    #                       received last (None before layer 0)
    #   (i, "gdn", proj, y) a GDN layer's in-projection rows [B, T, C + VD + 2 Hv] and its delta-rule
    #                       readout [B, T, Hv, Dv]
    #   (i, "mid", h, r)    the hidden rows once the mixer's branch r is added (the MLP's input)
    layer_probe = None

    # canvas blocks of at least this many (sequence, value head) pairs take the single-block MFMA readout
    # under "auto" (batch 64 x 16 heads: 30 vs 132-155 us per layer); smaller grids keep the token-recurrent
    # kernel (batch 1: 7.9 vs 10.4 us), whose verify rows are bitwise the AR rows
    GDR_BLOCK_MIN_HEADS = 128

    def _chunked_gdr(self, T: int, gdn_mode: int, B: int = 1, persist: bool = True) -> bool:
        c = self.cfg
        if self.gdr_form == "recurrent" or c.lin_k_dim not in (32, 64, 128) or c.lin_v_dim % 16:
            return False
        if self.gdr_form == "auto":
            block = (not persist and T <= 64 and c.lin_k_dim == 128 and c.lin_v_dim % 128 == 0
                     and B * c.lin_v_heads >= self.GDR_BLOCK_MIN_HEADS)
            return (gdn_mode == 1 and T > 64) or block
        return gdn_mode == 1 or T <= 64

    def _mm(self, x: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x @ w.T on hipBLASLt (torch.matmul): prefill chunks, batched steps and the LM head."""
        with K.timed("gemm"), self._choices:
            if out is None:
                return torch.matmul(x, w.t())
            return torch.matmul(x, w.t(), out=out)

    def _proj(self, s: "_Scratch", key: str, x: torch.Tensor, x_p: torch.Tensor, out_p: torch.Tensor,
              xf: Optional[torch.Tensor] = None):
        """One decoder projection of the N = B * T rows in x (x_p: the padded rows hipBLASLt reads; xf: the
        same rows in the weight-streaming GEMM's fragment order, when their producer wrote it).
        Returns the pending residual for add_norm when the projection feeds one (("parts", planes) from
        the weight-streaming GEMM, ("bf16", rows) from hipBLASLt), else None (output in out_p's rows)."""
        ws = self.ws.get(key) if s.N <= K.WS_MAX_M else None
        if ws is None:
            self._mm(x_p, self.w[key], out_p)
            return ("bf16", out_p[: s.N])
        wp, N, role, kg = ws
        with K.timed("ws_gemm"):
            if role == K.WS_PARTS:
                if xf is not None:
                    K.ws_gemm_frag(xf, s.N, wp, N, s.parts, epilogue=role)
                else:
                    K.ws_gemm(x, wp, N, s.parts, epilogue=role)
                return ("parts", kg)
            K.ws_gemm(x, wp, N, out_p, epilogue=role)
        return None

    def _proj_normed(self, s: "_Scratch", key: str, out_p: torch.Tensor, fused: bool) -> None:
        """A projection of the normed hidden rows: with `fused`, rmsnorm(h) inside the weight-streaming GEMM
        over h in fragment order (the norm weight is in the weight copy's columns; bf16 epilogue into out_p's
        rows, or the SwiGLU epilogue into s.actf in fragment order for the down projection); otherwise of x,
        which add_norm already normed."""
        if not fused:
            self._proj(s, key, s.x, s.x_p, out_p)
            return
        wp, N, role, _ = self.ws[key]
        with K.timed("ws_gemm"):
            if role == K.WS_SILU:
                K.ws_gemm_frag(s.hf, s.N, wp, N, s.actf, ss=s.ss, eps=self.cfg.rms_eps, epilogue=role, out_frag=True)
            else:
                K.ws_gemm_frag(s.hf, s.N, wp, N, out_p, ss=s.ss, eps=self.cfg.rms_eps, epilogue=role)

    def _residual(self, s: "_Scratch", pending) -> None:
        """h += the partial planes of the projection just run, and the sums of squares for the next norm."""
        with K.timed("residual"):
            K.residual_parts(s.h, s.parts, pending[1], s.ss, h_frag=s.hf)

    def _ws_silu(self, s: "_Scratch", p: str) -> bool:
        """True when the gate/up projection of layer prefix p runs with the SwiGLU epilogue here."""
        return s.N <= K.WS_MAX_M and p + "w_gu" in self.ws

    def _add_norm(self, s: "_Scratch", pending, w: torch.Tensor) -> None:
        """h += the pending residual (none before the first layer), x = rmsnorm(h) * (1 + w)."""
        eps = self.cfg.rms_eps
        with K.timed("add_rmsnorm"):
            if pending is not None and pending[0] == "parts":
                K.add_rmsnorm_parts(s.h, s.parts, pending[1], w, s.x, eps=eps)
            else:
                K.add_rmsnorm(s.h, None if pending is None else pending[1], w, s.x, eps=eps)

    def _branch(self, s: "_Scratch", pending) -> Optional[torch.Tensor]:
        """The residual branch `pending` as the bf16 rows [N, hidden] it adds to h (for the layer probe)."""
        if pending is None:
            return None
        if pending[0] == "bf16":
            return pending[1]
        return s.parts[: pending[1] * s.N * self.cfg.hidden].view(pending[1], s.N, -1).sum(0).to(torch.bfloat16)

    # a greedy verify of <= WS_MAX_M rows may run its LM head with the argmax epilogue (no logits written)
    fused_greedy_head = True

    def greedy_head_ok(self, rows: int) -> bool:
        """Whether forward(..., head="argmax") applies to a block of `rows` rows."""
        return self.fused_greedy_head and "lm_head" in self.ws and rows <= K.WS_MAX_M

    # a denoise pass of <= WS_MAX_M rows may read its argmax and confidence from the LM head's epilogue
    fused_draft_head = True

    def argmax_conf_ok(self) -> bool:
        """Whether forward(..., head="argmax_conf") applies (with greedy_head_ok for the row count): the LM
        head's column splits fit K.argmax_conf_splits."""
        if not (self.fused_draft_head and "lm_head" in self.ws):
            return False
        wp, V, _, _ = self.ws["lm_head"]
        return K.ws_argmax_splits(V, self.cfg.hidden) <= K.CONF_MAX_SPLITS

    def forward(self, ids: torch.Tensor, cache: SeqCache, mode: str, n_clean: int = 0,
                rows: Optional[int] = None, seq: Optional[slice] = None, row0: int = 0,
                logits_out: Optional[torch.Tensor] = None, head: str = "logits"):
        """One forward of a [B, T] block of token ids (device int64) on top of the cache.
        Returns bf16 logits [B, rows, V] of block rows row0 .. row0 + rows - 1 (default: every row; the
        LM head runs on those rows only). seq restricts the forward to a contiguous range of the
        cache's sequences (used by per-sequence prefill of ragged prompts). logits_out: a contiguous fp32
        [B, rows, V] buffer the LM head writes instead (its fp32 accumulators, no bf16 rounding); it is
        returned. head="argmax" (greedy_head_ok): the LM head reduces each row of its bf16 logits to one
        (max, first index) pair per column split instead of writing them; returns (pval, pidx)
        [B, rows, S] for K.greedy_accept_splits. head="argmax_conf": the same with each split's softmax
        denominator; returns (pval, pidx, psum) [B, rows, S] for K.argmax_conf_splits."""
        c, w = self.cfg, self.w
        B, T = ids.shape
        sq = seq if seq is not None else slice(0, cache.B)
        kv_k, kv_v = cache.kv_k[:, sq], cache.kv_v[:, sq]
        state, window = cache.state[:, sq], cache.window[:, sq]
        length, pos = cache.length[sq], cache.pos[sq]
        persist = mode == "causal"
        if mode in ("causal", "verify"):
            att_mask, gdn_mode, nc = K.MASK_VERIFY, 1, T
        elif mode == "canvas":
            att_mask, gdn_mode, nc = K.MASK_CANVAS, 2, n_clean
        elif mode == "draft":
            att_mask, gdn_mode, nc = K.MASK_DRAFT, 2, 1
        else:
            raise ValueError(f"unknown forward mode {mode!r}")
        s = self.scratch(B, T)
        N = B * T
        max_keys = min(cache.Lmax, cache.ctx_hint + T)
        fwd_timer = K.timed("forward").__enter__()
        torch.index_select(w["embed"], 0, ids.reshape(-1), out=s.h)
        # fused: every projection on the weight-streaming GEMM, each RMSNorm inside the GEMM that reads it
        # (residual_parts adds a projection's partial planes to h and leaves the sums of squares)
        fused = self.ws_fused and N <= K.WS_MAX_M
        if fused:
            with K.timed("residual"):
                K.residual_parts(s.h, None, 0, s.ss, h_frag=s.hf)
        pending = None  # the residual branch not yet added to h
        probe = self.layer_probe
        added = None    # the branch h received last (reported to the probe)
        for i in range(c.n_layers):
            p = f"l{i}."
            if not fused:
                self._add_norm(s, pending, w[p + "in_norm"])
                added = pending
            if probe is not None:  # h is complete here: layer i's input
                probe(i, "in", s.h, self._branch(s, added))
            j = self._slot[i]
            if c.is_attention(i):
                self._proj_normed(s, p + "w_qkv", s.qkv_p, fused)
                with K.timed("attn_prep"):
                    K.attn_prep(s.qkv, w[p + "q_norm"], w[p + "k_norm"], pos, length, s.q_att, kv_k[j], kv_v[j],
                                Hq=c.n_heads, Hkv=c.n_kv_heads, D=c.head_dim, rot_dim=c.rot_dim,
                                rope_theta=c.rope_theta, eps=c.rms_eps)
                # the q projection interleaves [q | gate] per head: gate (b, t, h, d) at h * 2D + D + d
                Wq = s.qkv.shape[2]
                gate = s.qkv.as_strided((B, T, c.n_heads, c.head_dim), (T * Wq, Wq, 2 * c.head_dim, 1),
                                        s.qkv.storage_offset() + c.head_dim)
                with K.timed("attn_canvas"):
                    if fused:  # straight into the output projection's fragment-order X
                        K.attn_canvas(s.q_att, kv_k[j], kv_v[j], length, mask_mode=att_mask, n_clean=nc, gate=gate,
                                      out=s.oattf, max_keys=max_keys, out_frag=True)
                    else:
                        K.attn_canvas(s.q_att, kv_k[j], kv_v[j], length, mask_mode=att_mask, n_clean=nc, gate=gate,
                                      out=s.o_att, max_keys=max_keys)
                pending = self._proj(s, p + "w_o", s.o_att_p[:N], s.o_att_p, s.r_p, xf=s.oattf if fused else None)
            else:
                self._proj_normed(s, p + "w_in", s.proj_p, fused)
                xv = s.proj[..., : c.conv_dim]
                off = c.conv_dim + c.value_dim
                b_in = s.proj[..., off: off + c.lin_v_heads]
                a_in = s.proj[..., off + c.lin_v_heads: off + 2 * c.lin_v_heads]
                rec = (s.q, s.k_rec[j], s.v_rec[j], s.g_rec[j], s.b_rec[j])
                chunked = self._chunked_gdr(T, gdn_mode, B, persist)
                keep = mode != "draft"  # a draft pass is never committed
                z = s.proj.view(N, -1)[:, c.conv_dim: c.conv_dim + c.value_dim]
                # the gated RMSNorm folded into the recurrence and the out projection (fused forward, one
                # staged chunk of rows)
                fold = (fused and self.fold_gnorm and s.gss is not None and not chunked and not self.fused_gdn
                        and T <= 40)
                if not chunked and self.fused_gdn and T <= 64 and c.lin_k_dim in (32, 64, 128):
                    with K.timed("gdn_fused"):
                        K.gdn_fused_layer(xv, window[j], w[p + "conv_w"], a_in, b_in, w[p + "A_log"],
                                          w[p + "dt_bias"], state[j], Hk=c.lin_k_heads, Hv=c.lin_v_heads,
                                          Dk=c.lin_k_dim, Dv=c.lin_v_dim, causal_mode=gdn_mode, num_clean=nc,
                                          state_out=state[j] if persist else None,
                                          rows_out=rec[1:] if keep else None,
                                          pre_out=s.pre_rec[j] if keep and not persist else None,
                                          window_out=s.win_tmp if persist else None, out=s.y)
                else:
                    with K.timed("gdn_prep"):
                        K.gdn_prep(xv, window[j], w[p + "conv_w"], a_in, b_in, w[p + "A_log"], w[p + "dt_bias"],
                                   Hk=c.lin_k_heads, Hv=c.lin_v_heads, Dk=c.lin_k_dim, Dv=c.lin_v_dim,
                                   window_out=s.win_tmp if persist else None,
                                   pre_out=s.pre_rec[j] if keep and not persist else None, out=rec)
                    if chunked:
                        with K.timed("gdr_chunk"):
                            K.gdr_chunk(s.q, s.k_rec[j], s.v_rec[j], s.g_rec[j], s.b_rec[j], state[j],
                                        causal_mode=gdn_mode, num_clean=nc, state_out=state[j] if persist else None,
                                        out=s.y)
                    elif fold:
                        with K.timed("gdr_recurrent"):
                            K.gdr_recurrent_gnorm(s.q, s.k_rec[j], s.v_rec[j], s.g_rec[j], s.b_rec[j], state[j],
                                                  z, w[p + "gnorm"], s.ynf, s.gss, causal_mode=gdn_mode,
                                                  num_clean=nc, state_out=state[j] if persist else None, out=s.y)
                    else:
                        with K.timed("gdr_recurrent"):
                            K.gdr_recurrent(s.q, s.k_rec[j], s.v_rec[j], s.g_rec[j], s.b_rec[j], state[j],
                                            causal_mode=gdn_mode, num_clean=nc,
                                            state_out=state[j] if persist else None, out=s.y)
                if persist:
                    window[j].copy_(s.win_tmp)
                if probe is not None:
                    probe(i, "gdn", s.proj, s.y)
                if fold:  # the recurrence left u and the sums of squares: the projection applies the norm
                    wp, Nout, _, _ = self.ws[p + "w_out"]
                    with K.timed("ws_gemm"):
                        kg = K.ws_gemm_headnorm(s.ynf, N, wp, Nout, s.gss, c.lin_v_heads, s.parts, eps=c.rms_eps)
                    pending = ("parts", kg)
                elif fused:  # straight into the out projection's fragment-order X
                    K.gated_rmsnorm(s.y.view(N, c.lin_v_heads, c.lin_v_dim), z, w[p + "gnorm"], s.ynf,
                                    eps=c.rms_eps, out_frag=True)
                    pending = self._proj(s, p + "w_out", s.yn_p[:N], s.yn_p, s.r_p, xf=s.ynf)
                else:
                    K.gated_rmsnorm(s.y.view(N, c.lin_v_heads, c.lin_v_dim), z, w[p + "gnorm"], s.yn, eps=c.rms_eps)
                    pending = self._proj(s, p + "w_out", s.yn_p[:N], s.yn_p, s.r_p)
            if fused:
                self._residual(s, pending)
                if probe is not None:  # the mixer's branch is in h
                    probe(i, "mid", s.h, self._branch(s, pending))
                self._proj_normed(s, p + "w_gu", s.act_p, fused)
            else:
                self._add_norm(s, pending, w[p + "post_norm"])
                if probe is not None:
                    probe(i, "mid", s.h, self._branch(s, pending))
                if self._proj(s, p + "w_gu", s.x, s.x_p, s.act_p if self._ws_silu(s, p) else s.gu_p) is not None:
                    K.silu_mul(s.gu, s.act)
            pending = self._proj(s, p + "w_down", s.act, s.act_p, s.r_p, xf=s.actf if fused else None)
            if fused:
                self._residual(s, pending)
                added, pending = pending, None
        self._add_norm(s, pending, w["final_norm"])
        if probe is not None:
            probe(c.n_layers, "in", s.h, self._branch(s, added if fused else pending))
        x = s.x.view(B, T, -1)
        if rows is not None or row0:
            x = x[:, row0: row0 + (rows if rows is not None else T - row0)]
        with K.timed("lm_head"):
            x2 = x.reshape(-1, x.shape[-1])
            wl = w.get("lm_head", w["embed"])
            if head in ("argmax", "argmax_conf"):
                if logits_out is not None or not self.greedy_head_ok(x2.shape[0]):
                    raise ValueError("forward: the argmax head needs the weight-streaming LM head and <= "
                                     f"{K.WS_MAX_M} rows")
                wp, V, _, _ = self.ws["lm_head"]
                conf = head == "argmax_conf"
                key = (head, x2.shape[0])
                bufs = self._head_bufs.get(key)
                if bufs is None:  # fixed addresses per row count (graph capture)
                    n = x2.shape[0] * K.ws_argmax_splits(V, x2.shape[1])
                    bufs = self._head_bufs[key] = tuple(
                        torch.empty(n, dtype=dt, device=self.dev)
                        for dt in ((torch.float32, torch.int32, torch.float32) if conf else (torch.float32, torch.int32)))
                if conf:
                    K.ws_gemm_argmax_conf(x2, wp, V, *bufs)
                else:
                    K.ws_gemm_argmax(x2, wp, V, *bufs)
                logits = tuple(t.view(B, x.shape[1], -1) for t in bufs)
            elif logits_out is not None:
                # fp32 logits straight from the GEMM's fp32 accumulators (no bf16 output widened again)
                if logits_out.dtype != torch.float32 or not logits_out.is_contiguous() \
                        or logits_out.numel() != x2.shape[0] * wl.shape[0]:
                    raise ValueError("forward: logits_out must be contiguous fp32 [B, rows, V]")
                with self._choices:
                    torch.ops.aten.mm.dtype_out(x2, wl.t(), torch.float32, out=logits_out.view(x2.shape[0], -1))
                logits = logits_out.view(B, x.shape[1], -1)
            elif x2.shape[0] <= K.WS_MAX_M and "lm_head" in self.ws:
                wp, V, _, _ = self.ws["lm_head"]
                logits = torch.empty(x2.shape[0], V, dtype=torch.bfloat16, device=self.dev)
                K.ws_gemm(x2, wp, V, logits, epilogue=K.WS_STORE)
                logits = logits.view(B, x.shape[1], -1)
            else:
                logits = self._mm(x2, wl).view(B, x.shape[1], -1)
        fwd_timer.__exit__(None, None, None)
        if persist:
            length += T
            pos += T
            if seq is None or cache.B == 1:
                cache.ctx_hint += T
            else:
                cache.ctx_hint = max(cache.ctx_hint, len(cache.tokens[sq.start]) + T)
        return logits

    # ---------------------------------------------------------------- reference API (batch 1 lists)
    def _ids(self, tokens, B: int = 1) -> torch.Tensor:
        t = torch.as_tensor(tokens, dtype=torch.int64)
        return t.reshape(B, -1).to(self.dev)

    def prefill(self, cache: SeqCache, tokens: list, seq: int = 0) -> torch.Tensor:
        """Causal prefill of `tokens` for sequence `seq` (chunked). Returns fp32 logits [V] of the last
        token (model.py:398-453)."""
        assert cache.pending is None and tokens
        logits = None
        sl = slice(seq, seq + 1)
        if len(cache.tokens[seq]) + len(tokens) > cache.Lmax:
            raise ValueError(f"KV cache capacity {cache.Lmax} exceeded by a prefill of {len(tokens)} tokens")
        for s0 in range(0, len(tokens), self.prefill_chunk):
            chunk = tokens[s0: s0 + self.prefill_chunk]
            logits = self.forward(self._ids(chunk), cache, "causal", seq=sl)
            cache.tokens[seq].extend(chunk)
            if self.progress_cb is not None:
                self.progress_cb(len(chunk))
        return logits[0, -1].float()

    def ar_step(self, cache: SeqCache, token: int) -> torch.Tensor:
        logits = self.forward(self._ids([token]), cache, "causal")
        cache.tokens[0].append(token)
        return logits[0, -1].float()

    def canvas(self, cache: SeqCache, canvas_tokens: list, n_clean: int, rows: Optional[int] = None,
               as_float: bool = True) -> torch.Tensor:
        """One self-spec canvas forward (model.py:472-484): rows < n_clean token-causal, MASK rows see
        the block. Returns logits [rows or blk, V] (shift readout). Call commit() afterwards."""
        assert cache.pending is None
        ids = self._ids(canvas_tokens)
        logits = self.forward(ids, cache, "canvas", n_clean=n_clean, rows=rows)
        cache.pending = {"tokens": [list(canvas_tokens)], "T": ids.shape[1]}
        return logits[0].float() if as_float else logits[0]

    def verify(self, cache: SeqCache, ids: torch.Tensor) -> torch.Tensor:
        """Token-causal pass over a [B, T] block (nothing persisted); commit() keeps a prefix."""
        assert cache.pending is None
        logits = self.forward(ids, cache, "verify")
        cache.pending = {"ids": ids, "T": ids.shape[1]}
        return logits

    def draft(self, cache: SeqCache, ids: torch.Tensor) -> torch.Tensor:
        """Block-diffusion denoising pass over a [B, T] block (nothing persisted, no commit)."""
        assert cache.pending is None
        return self.forward(ids, cache, "draft")

    def commit(self, cache: SeqCache, adv, tokens_host: Optional[list] = None) -> None:
        """Keep the first adv canvas rows (model.py:486-507): KV crop by length, GDN state advanced
        from the block-entry state by those rows, conv window rebuilt. adv: int (same for every
        sequence) or an int32 device tensor [B]. tokens_host: committed ids per sequence (host lists)
        when the caller already has them."""
        rec = cache.pending
        assert rec is not None
        T = rec["T"]
        B = cache.B
        if isinstance(adv, int):
            assert 1 <= adv <= T
            n_keep = torch.full((B,), adv, dtype=torch.int32, device=self.dev)
        else:
            n_keep = adv
        s = self.scratch(B, T)
        L = len(self.gdn_layers)
        if L:
            st = cache.state.view(L * B, *cache.state.shape[2:])
            win = cache.window.view(L * B, *cache.window.shape[2:])
            rows = (s.k_rec.view(L * B, *s.k_rec.shape[2:]), s.v_rec.view(L * B, *s.v_rec.shape[2:]),
                    s.g_rec.view(L * B, *s.g_rec.shape[2:]), s.b_rec.view(L * B, *s.b_rec.shape[2:]))
            pre = s.pre_rec.view(L * B, *s.pre_rec.shape[2:])
            with K.timed("gdn_restore"):
                if self._chunked_gdr(T, 1):
                    # every (layer, sequence) slot: the block-entry state advanced by its n_keep rows
                    K.gdr_chunk(None, *rows, st, state_out=st, n_keep=n_keep, want_out=False)
                    K.gdn_restore(n_keep, snap_window=win, window=win, preconv=pre)
                else:
                    K.gdn_restore(n_keep, snap_state=st, state=st, k=rows[0], v=rows[1], g=rows[2], beta=rows[3],
                                  snap_window=win, window=win, preconv=pre)
        cache.length += n_keep
        cache.pos += n_keep
        cache.ctx_hint += adv if isinstance(adv, int) else T
        if tokens_host is not None:
            for b in range(B):
                cache.tokens[b].extend(tokens_host[b])
        elif "tokens" in rec and isinstance(adv, int):
            for b in range(B):
                cache.tokens[b].extend(rec["tokens"][b][:adv])
        cache.pending = None


def build_runtime(cfg: HybridConfig, seed: int = 0, device="cuda:0", embed_scale: float = 1.0) -> TridaRuntime:
    """Random-init runtime: weights drawn on the device (no host copy of the 4B parameters)."""
    w = init_weights(cfg, seed=seed, device=device, embed_scale=embed_scale)
    return TridaRuntime(cfg, w, device=device)


def config_json(cfg: HybridConfig) -> str:
    return json.dumps(asdict(cfg))
