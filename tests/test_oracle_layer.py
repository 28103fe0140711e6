"""CPU pins of the oracle's layer compositions against transformers' own Qwen3_5GatedDeltaNet.

The reference runs its hot-path functions inside transformers' GatedDeltaNet layer (patched by
src/cb_engine.py:54-77) and in its own engine layer (src/cb_engine.py:318-352, src/cb_tp.py:153-263),
which restates that layer's sequence: in_proj -> conv -> split q|k|v -> gating -> repeat_interleave
-> gated delta rule -> gated norm -> out_proj.  Here the installed transformers layer, with random
weights, runs a fresh prompt, a continued prompt and cached decode steps through its own cache, and
the oracle's compositions (gdn_prefill_core, gdn_decode_core, gdn_gating, expand_key_heads) fed the
layer's projections and parameters must give the same outputs and states.  Mistakes planted in the
oracle (a and b swapped, the q|k split swapped, the h % r head map, z heads permuted) must fail the
same comparison.

Tolerances: the layer's prefill uses F.conv1d and torch's bf16 l2norm (which double-rounds in the
scalar tail of its loop), its decode uses F.conv1d where the reference's engine (and the oracle)
uses the elementwise window product (src/cb_engine.py:43-51): outputs agree to <= 2e-2 rel-L2 and
recurrent states to <= 1e-2, conv states bit for bit; every planted mistake moves the output or
the state by more than 0.1.
"""
import importlib

import pytest
import torch

from conftest import rel_l2

M = importlib.import_module("transformers.models.qwen3_5.modeling_qwen3_5")
from transformers.cache_utils import Cache, LinearAttentionLayer  # noqa: E402
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig  # noqa: E402

OUT_TOL, STATE_TOL, MUTANT_MIN = 2e-2, 1e-2, 0.1
HIDDEN = 64


def make_layer(Hk, Hv, D, seed=0):
    """A Qwen3_5GatedDeltaNet with random weights in bf16 (A_log, dt_bias, norm weight randomised
    too; projections scaled up so every term of the layer matters)."""
    torch.manual_seed(seed)
    cfg = Qwen3_5TextConfig(hidden_size=HIDDEN, linear_num_key_heads=Hk, linear_num_value_heads=Hv,
                            linear_key_head_dim=D, linear_value_head_dim=D, linear_conv_kernel_dim=4,
                            num_hidden_layers=1, layer_types=["linear_attention"], intermediate_size=64,
                            num_attention_heads=2, num_key_value_heads=1, head_dim=64, vocab_size=32,
                            rms_norm_eps=1e-6)
    m = M.Qwen3_5GatedDeltaNet(cfg, 0)
    with torch.no_grad():
        m.dt_bias.copy_(torch.randn(Hv))
        m.A_log.copy_(torch.log(torch.rand(Hv) * 0.5 + 0.05))
        m.norm.weight.copy_(1 + 0.1 * torch.randn(D))
        m.conv1d.weight.mul_(3.0)
        for lin in (m.in_proj_qkv, m.in_proj_z, m.in_proj_a, m.in_proj_b):
            lin.weight.mul_(4.0)
    return m.to(torch.bfloat16).eval()


def run_layer(m, h, splits):
    """The layer's own forward through a transformers cache: h [1, L, hidden] fed in pieces
    (prompt chunks of any length, then single tokens = cached decode).  Returns the outputs
    [L, hidden] and (conv state, recurrent state) after every piece."""
    cache = Cache(layers=[LinearAttentionLayer()])
    outs, states = [], []
    with torch.no_grad():
        for lo, hi in splits:
            outs.append(m(h[:, lo:hi], cache_params=cache)[0])
            L = cache.layers[0]
            states.append((L.conv_states[0].clone(), L.recurrent_states[0].clone()))
    return torch.cat(outs, 0), states


def layer_inputs(m, h):
    """The layer's projections (not part of the oracle) and parameters, as the engine feeds them."""
    with torch.no_grad():
        x = h[0]
        return dict(mixed=m.in_proj_qkv(x), z=m.in_proj_z(x), b=m.in_proj_b(x), a=m.in_proj_a(x),
                    cw=m.conv1d.weight.squeeze(1).detach(), A_log=m.A_log.detach(), dt=m.dt_bias.detach(),
                    nw=m.norm.weight.detach())


def oracle_prefill(oracle, m, p, lo, hi, hist=None, init=None, **over):
    q = dict(p, **over)
    with torch.no_grad():
        core, cs, rs = oracle.gdn_prefill_core(q["mixed"][lo:hi], q["z"][lo:hi], q["a"][lo:hi], q["b"][lo:hi], q["cw"],
                                               q["A_log"], q["dt"], q["nw"], m.num_k_heads, m.num_v_heads,
                                               m.head_k_dim, conv_history=hist, initial_state=init)
        return m.out_proj(core), cs, rs


def oracle_decode(oracle, m, p, t, cs, rs):
    with torch.no_grad():
        core = oracle.gdn_decode_core(p["mixed"][t:t + 1], p["z"][t:t + 1], p["a"][t:t + 1], p["b"][t:t + 1], cs,
                                      p["cw"], p["A_log"], p["dt"], p["nw"], rs, m.num_k_heads, m.num_v_heads,
                                      m.head_k_dim)
        return m.out_proj(core)


@pytest.mark.parametrize("Hk,Hv", [(2, 4), (2, 6)])
def test_layer_compositions_match_transformers(oracle, Hk, Hv):
    """Fresh prompt (77 tokens), continued prompt (+40 tokens from the cached conv window and
    recurrent state), then 3 cached decode steps: outputs and both states after each piece."""
    D, T1, T2, steps = 32, 77, 40, 3
    m = make_layer(Hk, Hv, D)
    h = torch.randn(1, T1 + T2 + steps, HIDDEN).to(torch.bfloat16)
    T = T1 + T2
    splits = [(0, T1), (T1, T)] + [(T + s, T + s + 1) for s in range(steps)]
    ref, states = run_layer(m, h, splits)
    p = layer_inputs(m, h)
    o1, cs, rs = oracle_prefill(oracle, m, p, 0, T1)
    assert rel_l2(o1, ref[:T1]) <= OUT_TOL
    assert torch.equal(cs[0], states[0][0][0]) and rel_l2(rs, states[0][1]) <= STATE_TOL
    o2, cs, rs = oracle_prefill(oracle, m, p, T1, T, hist=cs, init=rs)
    assert rel_l2(o2, ref[T1:T]) <= OUT_TOL
    assert torch.equal(cs[0], states[1][0][0]) and rel_l2(rs, states[1][1]) <= STATE_TOL
    cs, rs = cs.clone(), rs.clone()
    for s in range(steps):
        o = oracle_decode(oracle, m, p, T + s, cs, rs)
        assert rel_l2(o, ref[T + s:T + s + 1]) <= OUT_TOL
        assert torch.equal(cs, states[2 + s][0]) and rel_l2(rs, states[2 + s][1]) <= STATE_TOL


def _mutant_errors(oracle, Hk, Hv, mutate):
    D, T = 32, 70
    m = make_layer(Hk, Hv, D, seed=1)
    h = torch.randn(1, T + 1, HIDDEN).to(torch.bfloat16)
    ref, states = run_layer(m, h, [(0, T), (T, T + 1)])
    p = layer_inputs(m, h)
    with mutate(oracle, p, Hk, D) as over:
        o, cs, rs = oracle_prefill(oracle, m, p, 0, T, **over)
        od = oracle_decode(oracle, m, dict(p, **over), T, cs.clone(), rs.clone())
    return max(rel_l2(o, ref[:T]), rel_l2(rs, states[0][1]), rel_l2(od, ref[T:]))


class _Swap:
    """Context managers that plant one mistake each in the oracle's composition."""

    def __init__(self, fn):
        self.fn = fn

    def __call__(self, oracle, p, Hk, D):
        self.args = (oracle, p, Hk, D)
        return self

    def __enter__(self):
        return self.fn(*self.args, self)

    def __exit__(self, *exc):
        if hasattr(self, "restore"):
            self.restore()
        return False


def _ab_swapped(oracle, p, Hk, D, ctx):
    return dict(a=p["b"], b=p["a"])


def _qk_swapped(oracle, p, Hk, D, ctx):
    kd = Hk * D
    x = p["mixed"]
    return dict(mixed=torch.cat([x[:, kd:2 * kd], x[:, :kd], x[:, 2 * kd:]], 1),
                cw=torch.cat([p["cw"][kd:2 * kd], p["cw"][:kd], p["cw"][2 * kd:]], 0))


def _head_map_mod(oracle, p, Hk, D, ctx):
    orig = oracle.expand_key_heads
    oracle.expand_key_heads = lambda x, r: x.repeat(1, 1, r, 1) if r > 1 else x   # value head h -> key h % Hk
    ctx.restore = lambda: setattr(oracle, "expand_key_heads", orig)
    return {}


def _z_heads_permuted(oracle, p, Hk, D, ctx):
    z = p["z"]
    return dict(z=z.reshape(z.shape[0], -1, D).flip(1).reshape(z.shape[0], -1))


@pytest.mark.parametrize("name,fn", [("a<->b", _ab_swapped), ("q<->k split", _qk_swapped),
                                     ("h % r head map", _head_map_mod), ("z heads permuted", _z_heads_permuted)])
def test_planted_composition_mistake_is_caught(oracle, name, fn):
    err = _mutant_errors(oracle, 2, 4, _Swap(fn))
    assert err > MUTANT_MIN, f"transformers pin missed the planted mistake '{name}' (error {err:.2e})"
    # and the unmutated oracle passes the same comparison
    assert _mutant_errors(oracle, 2, 4, _Swap(lambda *a: {})) <= OUT_TOL


def test_gating_matches_transformers_layer(oracle):
    """beta and g exactly as the layer forms them from b and a (HF:497-498)."""
    m = make_layer(2, 4, 32, seed=2)
    x = torch.randn(50, HIDDEN).to(torch.bfloat16)
    with torch.no_grad():
        a, b = m.in_proj_a(x), m.in_proj_b(x)
        beta_ref = b.sigmoid()
        g_ref = -m.A_log.float().exp() * torch.nn.functional.softplus(a.float() + m.dt_bias)
        beta, g = oracle.gdn_gating(a, b, m.A_log, m.dt_bias)
    assert torch.equal(beta, beta_ref) and torch.equal(g, g_ref)


def test_prefill_core_empty_prompt(oracle):
    """An empty prompt in a packed batch: no outputs, its conv state is its history and its recurrent
    state its initial state, bit for bit; the prompts around it are unchanged by its presence."""
    D, Hk, Hv, K = 16, 2, 4, 4
    C = (2 * Hk + Hv) * D
    g_ = torch.Generator().manual_seed(5)
    lens = [7, 0, 20]
    T = sum(lens)
    mixed = torch.randn(T, C, generator=g_).to(torch.bfloat16)
    z = torch.randn(T, Hv * D, generator=g_).to(torch.bfloat16)
    a = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    b = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    cw = (0.5 * torch.randn(C, K, generator=g_)).to(torch.bfloat16)
    A_log, dt, nw = torch.randn(Hv, generator=g_), torch.randn(Hv, generator=g_), torch.ones(D)
    hist = torch.randn(3, C, K, generator=g_).to(torch.bfloat16)
    s0 = 0.1 * torch.randn(3, Hv, D, D, generator=g_)
    cu = torch.tensor([0, 7, 7, 27], dtype=torch.int32)
    core, conv, rec = oracle.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D, cu_seqlens=cu,
                                              conv_history=hist, initial_state=s0)
    assert core.shape == (T, Hv * D)
    assert torch.equal(conv[1], hist[1]) and torch.equal(rec[1], s0[1])
    keep = torch.tensor([0, 2])
    cu2 = torch.tensor([0, 7, 27], dtype=torch.int32)
    core2, conv2, rec2 = oracle.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D, cu_seqlens=cu2,
                                                 conv_history=hist[keep], initial_state=s0[keep])
    assert torch.equal(core, core2) and torch.equal(conv[keep], conv2) and torch.equal(rec[keep], rec2)
