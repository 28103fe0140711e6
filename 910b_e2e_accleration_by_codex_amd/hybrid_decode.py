"""Hybrid (GDN + full-attention) decode step of a Qwen3.5-shaped model, graph-captured.

The decode side of the reference's engine (src/cb_engine.py:123-187 graph capture, :246-250 dense
decode over all slots, :318-352 the GDN layer) for a whole layer stack: every GDN layer runs its
in-projections as one GEMM, the fused HIP decode core (conv update + gating + l2norm + recurrent
step + gated RMSNorm, one kernel) and out_proj; every fourth layer is GQA full attention
(HF Qwen3_5Attention: gated q, per-head q/k RMSNorm, partial rotary, modeling_qwen3_5.py) over a
per-slot KV cache; each layer ends with the SwiGLU MLP.  Weights are random (no checkpoints), the
slots' GDN states and KV caches are pre-filled with random values at per-slot context lengths.

The GDN layer core, every linear of the step (the weight-streaming decode projection kernel,
gdn_decode_linear), the residual adds with their RMSNorms and the SwiGLU products are this library's
kernels; the output projections hand their split-K partial sums straight to the residual add + norm,
and gate_up its partials to SwiGLU.  The attention layer (q/k norms, rotary, cache writes, softmax
attention, gate) is this library's three-launch decode attention.  The KV cache keeps K transposed
([slot, kv head, head_dim, position]) so the score loads run along positions.
"""
from dataclasses import dataclass
from types import SimpleNamespace

import torch

from .cb_engine import (GDNSlots, PackedWeight, add_rms_norm, attn_decode_workspace, decode_linear, decode_linear_partial,
                        gdn_decode_core, gqa_decode_attention, swiglu)


@dataclass
class HybridConfig:
    """Layer shapes.  The defaults are Qwen3.5-27B's (src/cb_tp.py:7-10, HF configuration_qwen3_5.py):
    hidden 5120, 64 layers with every fourth one full attention, GDN H_k=16 / H_v=48 / d=128 with a
    4-tap conv, attention 24 q / 4 kv heads of 256 with a quarter of each head rotary, MLP 17408."""
    hidden: int = 5120
    layers: int = 64
    full_every: int = 4  # 0: GDN layers only
    gdn_k_heads: int = 16
    gdn_v_heads: int = 48
    gdn_head: int = 128
    conv_k: int = 4
    attn_heads: int = 24
    kv_heads: int = 4
    attn_head: int = 256
    rotary_frac: float = 0.25
    rope_theta: float = 10000.0
    mlp: int = 17408     # 0: no MLP (the token mixers alone)
    vocab: int = 248320  # 0: no LM head (the step returns the final hidden state)
    eps: float = 1e-6

    def is_full(self, i):
        return self.full_every > 0 and (i + 1) % self.full_every == 0

    @property
    def conv_dim(self):
        return (2 * self.gdn_k_heads + self.gdn_v_heads) * self.gdn_head


class HybridDecoder:
    """Random-weight hybrid stack with slot state for ``n_slots`` sequences.  ``ctx`` (int [N], host)
    are the per-slot context lengths already in the caches; each ``step`` appends one token per slot.
    Every linear weight is packed once for the decode projection kernel (``L.<name>_p``); the plain
    [N, K] weights are kept only with ``keep_plain`` (for checks against a reference)."""

    def __init__(self, cfg, n_slots, ctx, max_steps, device, seed=0, weight_std=0.02, keep_plain=False):
        self.cfg, self.N, self.dev = cfg, n_slots, device
        g_ = torch.Generator(device=device).manual_seed(seed)
        bf = torch.bfloat16

        def w(*shape, std=weight_std):
            return (torch.randn(*shape, generator=g_, device=device) * std).to(bf)

        H, D = cfg.hidden, cfg.gdn_head
        self.layers = []
        gdn_ids = [i for i in range(cfg.layers) if not cfg.is_full(i)]
        self.slots = GDNSlots(n_slots, gdn_ids, cfg.conv_dim, cfg.conv_k, cfg.gdn_v_heads, D, device)
        ctx = torch.as_tensor(ctx, dtype=torch.int64)
        self.max_ctx = (int(ctx.max()) + max_steps + 3) // 4 * 4  # the attention kernels read 4 positions at once
        self.pos = ctx.to(device=device, dtype=torch.int64)  # position of the next token per slot
        kv, hd = cfg.kv_heads, cfg.attn_head
        for i in range(cfg.layers):
            L = SimpleNamespace(full=cfg.is_full(i), in_norm=w(H), post_norm=w(H),
                                gate_up=w(2 * cfg.mlp, H) if cfg.mlp else None,
                                down=w(H, cfg.mlp) if cfg.mlp else None, gate_up_p=None)
            if L.full:
                L.qkv = w(cfg.attn_heads * hd * 2 + 2 * kv * hd, H)
                L.o = w(H, cfg.attn_heads * hd)
                L.q_norm, L.k_norm = w(hd), w(hd)
                # cache: K transposed [N, kv, hd, T], V [N, kv, T, hd]; random history below each ctx
                L.kt = torch.randn(n_slots, kv, hd, self.max_ctx, generator=g_, device=device).to(bf)
                L.v = torch.randn(n_slots, kv, self.max_ctx, hd, generator=g_, device=device).to(bf)
            else:
                Hv, Hk, C = cfg.gdn_v_heads, cfg.gdn_k_heads, cfg.conv_dim
                L.in_proj = w(C + Hv * D + 2 * Hv, H)  # in_proj_qkv | in_proj_z | in_proj_b | in_proj_a
                L.conv_w = (0.5 * torch.randn(C, cfg.conv_k, generator=g_, device=device)).to(bf)
                L.A_log = torch.full((Hv,), -2.302585092994046, device=device)
                L.dt_bias = torch.full((Hv,), 2.0, device=device)
                L.norm_w = (1 + 0.02 * torch.randn(D, generator=g_, device=device)).to(bf)
                L.out = w(H, Hv * D)
                self.slots.conv[i].copy_(torch.randn(n_slots, C, cfg.conv_k, generator=g_, device=device).to(bf))
                self.slots.rec[i].copy_(0.02 * torch.randn(n_slots, Hv, D, D, generator=g_, device=device))
            for name in ("in_proj", "out", "qkv", "o", "gate_up", "down"):
                wt = getattr(L, name, None)
                if wt is not None:
                    setattr(L, name + "_p", PackedWeight(wt))
                    if not keep_plain:
                        setattr(L, name, None)
            self.layers.append(L)
        self.final_norm = w(H)
        self.lm_head = w(cfg.vocab, H) if cfg.vocab else None
        self.lm_head_p = PackedWeight(self.lm_head) if cfg.vocab else None
        if not keep_plain:
            self.lm_head = None
        rd = int(hd * cfg.rotary_frac)
        self.rotary_dim = rd
        self.inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, rd, 2, device=device, dtype=torch.float32) / rd))
        self.attn_work = (attn_decode_workspace(n_slots, cfg.attn_heads, hd, self.max_ctx, device)
                          if any(L.full for L in self.layers) else None)

    # -- layers ------------------------------------------------------------------------------
    def gdn(self, i, L, x, partial=False):
        cfg, n = self.cfg, x.shape[0]
        Hv, D, C = cfg.gdn_v_heads, cfg.gdn_head, cfg.conv_dim
        proj = decode_linear(x, L.in_proj_p)           # one product for qkv | z | b | a
        mixed = proj[:, :C]
        z = proj[:, C:C + Hv * D]
        b = proj[:, C + Hv * D:C + Hv * D + Hv]
        a = proj[:, C + Hv * D + Hv:]
        core = gdn_decode_core(mixed, z, a, b, self.slots.conv[i], L.conv_w, L.A_log, L.dt_bias, L.norm_w,
                               self.slots.rec[i], cfg.gdn_k_heads, Hv, D, cfg.eps)
        return (decode_linear_partial if partial else decode_linear)(core.reshape(n, Hv * D), L.out_p)

    def attention(self, L, x, partial=False):
        cfg = self.cfg
        nh, kv, hd = cfg.attn_heads, cfg.kv_heads, cfg.attn_head
        proj = decode_linear_partial(x, L.qkv_p)   # per head q | gate, then k, then v: split-K partials
        # q/k norms, partial rotary, the cache writes at each slot's position, softmax attention and
        # the sigmoid gate: three HIP launches
        o = gqa_decode_attention(proj, self.pos, L.q_norm, L.k_norm, self.inv_freq, L.kt, L.v, nh, kv, hd,
                                 self.rotary_dim, cfg.eps, work=self.attn_work)
        return (decode_linear_partial if partial else decode_linear)(o, L.o_p)

    def mlp(self, L, x, partial=False):
        act = swiglu(decode_linear_partial(x, L.gate_up_p))
        return (decode_linear_partial if partial else decode_linear)(act, L.down_p)

    def step(self, h):
        """h [N, hidden] bf16 (the step's token embeddings) -> logits [N, vocab] (or the final hidden
        state without an LM head).  Advances every slot by one token.  Each residual add is fused
        with the RMSNorm that follows it (Qwen3_5DecoderLayer.forward's order)."""
        eps = self.cfg.eps
        norms = []
        for L in self.layers:
            norms.append(L.in_norm)
            if L.gate_up_p is not None:
                norms.append(L.post_norm)
        norms.append(self.final_norm)
        h, x = add_rms_norm(h, None, norms[0], eps)
        k = 1
        for i, L in enumerate(self.layers):
            # the token mixer's and the MLP's output projections hand their split-K partial sums
            # straight to the residual add + norm
            mix = self.attention(L, x, partial=True) if L.full else self.gdn(i, L, x, partial=True)
            h, x = add_rms_norm(h, mix, norms[k], eps)
            k += 1
            if L.gate_up_p is not None:
                h, x = add_rms_norm(h, self.mlp(L, x, partial=True), norms[k], eps)
                k += 1
        self.pos += 1
        return decode_linear(x, self.lm_head_p) if self.lm_head_p is not None else x


class HybridDecodeGraph:
    """The whole decode step captured once as a HIP graph and replayed (src/cb_engine.py:123-187):
    ``inp`` is the static input buffer, ``replay()`` returns the static output."""

    def __init__(self, model, inp):
        self.model, self.inp = model, inp
        self.graph = torch.cuda.CUDAGraph()
        dev = inp.device
        stream = torch.cuda.Stream(device=dev)
        stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(stream):
            model.step(inp)  # warm-up (advances the slots by one token)
        torch.cuda.current_stream(dev).wait_stream(stream)
        torch.cuda.synchronize(dev)
        with torch.cuda.graph(self.graph):
            self.out = model.step(inp)

    def replay(self):
        self.graph.replay()
        return self.out
