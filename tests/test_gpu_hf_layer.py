"""GPU: the drop-in boundary through transformers' own Qwen3_5GatedDeltaNet.

patch_model (src/cb_engine.py:54-77) installs this library's functions on a GatedDeltaNet layer
(and on the module-level names transformers >= 5.6 calls); the patched layer then runs a fresh
prompt, a continued prompt and cached decode steps through its own cache on the GPU.  It is checked
against
  * the unpatched layer on the GPU (torch's own ops): outputs, conv state bit for bit, recurrent
    state;
  * the oracle's compositions fed the layer's projections and parameters (the reference's
    equivalence test compares tokens and GDN state, scripts/test_chunked_prefill_cpu.py:86-90).
The engine-side decode layer gdn_decode_layer (src/cb_engine.py:318-352) is checked against the
layer's own cached decode forward.

Tolerances: outputs <= 1e-2 rel-L2, recurrent states <= 1e-3 against the oracle; against the
unpatched layer the decode conv differs in form (F.conv1d there, the reference's elementwise window
product here, src/cb_engine.py:43-51, HANDOFF.md:136), so decode outputs and states are held to
2e-2 / 1e-2 there.
"""
import importlib

import pytest
import torch

from conftest import rel_l2
from test_oracle_layer import HIDDEN, layer_inputs, make_layer, oracle_decode, oracle_prefill, run_layer

M = importlib.import_module("transformers.models.qwen3_5.modeling_qwen3_5")
_NAMES = ("torch_chunk_gated_delta_rule", "torch_recurrent_gated_delta_rule", "causal_conv1d_update")


@pytest.fixture
def restore_transformers():
    saved = {n: getattr(M, n) for n in _NAMES}
    yield
    for n, f in saved.items():
        setattr(M, n, f)


def _patched_copy(gdn, m, dev):
    import copy
    pm = copy.deepcopy(m).to(dev)
    gdn.patch_model(torch.nn.ModuleList([pm]), fast_gdn=True, gdn_v2=True)
    return pm


@pytest.mark.gpu
@pytest.mark.parametrize("Hk,Hv", [(2, 4), (2, 6)])
def test_patched_layer_matches_unpatched_and_oracle(gdn, oracle, dev, restore_transformers, Hk, Hv):
    D, T1, T2, steps = 128, 150, 70, 3
    m = make_layer(Hk, Hv, D, seed=3)
    g_ = torch.Generator().manual_seed(4)
    h = torch.randn(1, T1 + T2 + steps, HIDDEN, generator=g_).to(torch.bfloat16)
    T = T1 + T2
    splits = [(0, T1), (T1, T)] + [(T + s, T + s + 1) for s in range(steps)]
    # unpatched layer on the GPU first (patching rebinds transformers' module-level names)
    md = m.to(dev)
    ref, ref_states = run_layer(md, h.to(dev), splits)
    # the layer's projections as the GPU forms them (the conv state holds them bit for bit)
    p = {k: v.cpu() for k, v in layer_inputs(md, h.to(dev)).items()}
    pm = _patched_copy(gdn, m, dev)
    assert M.torch_chunk_gated_delta_rule is gdn.fast_chunk_gated_delta_rule_v2
    out, states = run_layer(pm, h.to(dev), splits)
    torch.cuda.synchronize()
    # against the unpatched layer
    assert rel_l2(out[:T], ref[:T]) <= 1e-2
    assert rel_l2(out[T:], ref[T:]) <= 2e-2
    for i, ((c, r), (cr, rr)) in enumerate(zip(states, ref_states)):
        assert torch.equal(c, cr), f"conv state after piece {i}"
        assert rel_l2(r, rr) <= (1e-3 if i < 2 else 1e-2), f"recurrent state after piece {i}"
    # against the oracle's compositions fed the same projections (the oracle runs on the CPU)
    mc = m.cpu()
    o1, cs, rs = oracle_prefill(oracle, mc, p, 0, T1)
    o2, cs, rs2 = oracle_prefill(oracle, mc, p, T1, T, hist=cs, init=rs)
    assert rel_l2(out[:T1], o1) <= 1e-2 and rel_l2(out[T1:T], o2) <= 1e-2
    assert rel_l2(states[0][1], rs) <= 1e-3 and rel_l2(states[1][1], rs2) <= 1e-3
    assert torch.equal(states[1][0].cpu(), cs)
    cs, rs2 = cs.clone(), rs2.clone()
    for s in range(steps):
        o = oracle_decode(oracle, mc, p, T + s, cs, rs2)
        assert rel_l2(out[T + s:T + s + 1], o) <= 1e-2
        assert torch.equal(states[2 + s][0].cpu(), cs) and rel_l2(states[2 + s][1], rs2) <= 1e-3


@pytest.mark.gpu
def test_gdn_decode_layer_matches_layer_forward(gdn, dev, restore_transformers):
    """CBEngine._gdn's decode sequence (gdn_decode_layer: projections, the fused HIP core with the
    states updated in place, out_proj) equals the layer's own cached decode step on 5 slots."""
    Hk, Hv, D, T, N = 2, 4, 128, 40, 5
    m = make_layer(Hk, Hv, D, seed=5).to(dev)
    g_ = torch.Generator().manual_seed(6)
    h = torch.randn(N, T + 2, HIDDEN, generator=g_).to(torch.bfloat16).to(dev)
    from transformers.cache_utils import Cache, LinearAttentionLayer
    cache = Cache(layers=[LinearAttentionLayer()])
    with torch.no_grad():
        m(h[:, :T], cache_params=cache)
        conv = cache.layers[0].conv_states[0].clone().contiguous()
        rec = cache.layers[0].recurrent_states[0].clone().contiguous().float()
        outs = []
        for s in range(2):
            outs.append(gdn.gdn_decode_layer(m, h[:, T + s:T + s + 1], conv, rec))
        gdn.patch_model(torch.nn.ModuleList([m]), fast_gdn=True, gdn_v2=True)
        ref = [m(h[:, T + s:T + s + 1], cache_params=cache) for s in range(2)]
    torch.cuda.synchronize()
    for s in range(2):
        assert rel_l2(outs[s], ref[s]) <= 1e-2
    assert torch.equal(conv, cache.layers[0].conv_states[0])
    assert rel_l2(rec, cache.layers[0].recurrent_states[0]) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("H", [64, 256, 1000, 5120])
def test_patched_rmsnorm_matches_hf(gdn, dev, H):
    """patch_model's fused Qwen3_5RMSNorm (src/cb_engine.py:62-63) against transformers' own forward
    on the GPU: within one bf16 ulp everywhere (the sum of squares is taken in another order) and
    mostly exact; 3-D rows, and a non-contiguous input like q_norm's half of the fused q|gate
    projection.  H = 1000 takes the element-loop kernel, the others the 16-byte one."""
    import copy
    g_ = torch.Generator().manual_seed(H)
    ref = M.Qwen3_5RMSNorm(H, eps=1e-6)
    with torch.no_grad():
        ref.weight.copy_(0.1 * torch.randn(H, generator=g_))
    ref = ref.to(dev, torch.bfloat16)
    pat = copy.deepcopy(ref)
    gdn.patch_model(torch.nn.ModuleList([pat]))
    assert pat.forward.__func__ is gdn.fused_rmsnorm
    x = (3 * torch.randn(2, 37, H, generator=g_)).to(torch.bfloat16).to(dev)
    qg = (3 * torch.randn(3, 5, 2, 2 * H, generator=g_)).to(torch.bfloat16).to(dev)
    xs = torch.chunk(qg, 2, dim=-1)[0]          # [3, 5, 2, H], rows strided by 2H
    for inp in (x, xs):
        with torch.no_grad():
            y_ref, y = ref(inp), pat(inp)
        torch.cuda.synchronize()
        assert y.shape == inp.shape and y.dtype == torch.bfloat16
        diff = (y.float() - y_ref.float()).abs()
        ulp = y_ref.float().abs().clamp_min(2 ** -126) * 2 ** -7
        assert (diff <= ulp).all(), "fused RMSNorm off by more than one bf16 ulp"
        assert (diff == 0).float().mean() >= 0.98
