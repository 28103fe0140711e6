"""GPU parity at the workload shapes themselves (H_k=16, H_v=32 or 48, d=128):

  * varlen packed prefill layer, 16 prompts with seeded lengths uniform in [200, 1500] (14,806
    tokens), random initial states, zero and random conv history -- the fused layer
    (gdn_prefill_core) against the oracle's composition (src/cb_tp.py:153-181, :230-263);
  * one long sequence, T = 32768, the chunked rule (src/gdn_chunk_fast2.py:11-62) at full width,
    output and final state of every value head against the oracle;
  * the chunked rule at Qwen3.5-27B's GDN shape (H_v = 48) at T = 8192, seven value heads, and the
    fused prefill layer at that shape (conv 10240 x 4) over 4 packed prompts, every head;
  * the Qwen3.5-27B-shaped decode step (48 GDN + 16 attention layers, hidden 5120, H_v = 48, 16
    slots, contexts uniform in [512, 4096]): graph replays equal eager steps over three steps, and
    one GDN layer at that shape (projections, fused core, out_proj) against the oracle's core.
Tolerances: outputs rel-L2 <= 1e-2, fp32 states <= 1e-3, conv states bit for bit.
"""
import importlib

import pytest
import torch

from conftest import PKG_NAME, rel_l2

OUT_TOL, STATE_TOL = 1e-2, 1e-3
HK, HV, D, K = 16, 32, 128, 4
C = (2 * HK + HV) * D


def varlen_layer_inputs(seed=2):
    """The varlen workload: lengths torch.randint(200, 1501, (16,)) from seed 2, then pre-conv
    mixed_qkv, z, a, b ~ N(0, 1) bf16, conv weight 0.5 N(0, 1), A_log = log 0.1, dt_bias = 2 (so
    g = -0.1 softplus(a + 2), beta = sigmoid(b)), norm weight 1 + 0.02 N(0, 1), S0 ~ N(0, 0.02)."""
    g_ = torch.Generator().manual_seed(seed)
    lens = torch.randint(200, 1501, (16,), generator=g_)
    cu = torch.zeros(17, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    T = int(cu[-1])
    bf = torch.bfloat16
    x = dict(mixed=torch.randn(T, C, generator=g_).to(bf), z=torch.randn(T, HV * D, generator=g_).to(bf),
             a=torch.randn(T, HV, generator=g_).to(bf), b=torch.randn(T, HV, generator=g_).to(bf),
             cw=(0.5 * torch.randn(C, K, generator=g_)).to(bf), A_log=torch.full((HV,), -2.302585092994046),
             dt=torch.full((HV,), 2.0), nw=(1 + 0.02 * torch.randn(D, generator=g_)).to(bf),
             s0=0.02 * torch.randn(16, HV, D, D, generator=g_),
             hist=torch.randn(16, C, K, generator=g_).to(bf))
    return cu, x


@pytest.mark.gpu
@pytest.mark.parametrize("history", [False, True])
def test_varlen_prefill_layer_16_prompts(gdn, oracle, dev, history):
    cu, x = varlen_layer_inputs()
    assert int(cu[-1]) == 14806
    hist = x["hist"] if history else None
    ref_core, ref_conv, ref_rec = oracle.gdn_prefill_core(x["mixed"], x["z"], x["a"], x["b"], x["cw"], x["A_log"],
                                                          x["dt"], x["nw"], HK, HV, D, cu_seqlens=cu,
                                                          conv_history=hist, initial_state=x["s0"])
    d = {k: v.to(dev) for k, v in x.items()}
    core, conv, rec = gdn.gdn_prefill_core(d["mixed"], d["z"], d["a"], d["b"], d["cw"], d["A_log"], d["dt"], d["nw"],
                                           HK, HV, D, cu_seqlens=cu, conv_history=d["hist"] if history else None,
                                           initial_state=d["s0"])
    torch.cuda.synchronize()
    assert torch.equal(conv.cpu(), ref_conv)
    assert rel_l2(core, ref_core) <= OUT_TOL
    for s in range(16):
        assert rel_l2(rec[s], ref_rec[s]) <= STATE_TOL, f"sequence {s}"
        lo, hi = int(cu[s]), int(cu[s + 1])
        assert rel_l2(core[lo:hi], ref_core[lo:hi]) <= OUT_TOL, f"sequence {s}"


@pytest.mark.gpu
def test_prefill_layer_model_shape_Hv48(gdn, oracle, dev):
    """The fused prefill layer at Qwen3.5-27B's GDN shape (H_k=16, H_v=48, d=128, conv 10240 x 4; the
    reference model, src/cb_tp.py:7-10): 4 packed prompts (353 tokens -- the reference's published prefill
    size --, 1000, 64 and 517) with conv history, initial states, and per-head decays from slow to fast
    (exp(A_log) from 0.002 to 2), against the oracle's composition: conv states exact, outputs within
    1e-2 and states within 1e-3 per prompt."""
    Hk, Hv, K = 16, 48, 4
    C = (2 * Hk + Hv) * D
    lens = [353, 1000, 64, 517]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T = int(cu[-1])
    g_ = torch.Generator().manual_seed(27)
    bf = torch.bfloat16
    x = dict(mixed=torch.randn(T, C, generator=g_).to(bf), z=torch.randn(T, Hv * D, generator=g_).to(bf),
             a=torch.randn(T, Hv, generator=g_).to(bf), b=torch.randn(T, Hv, generator=g_).to(bf),
             cw=(0.5 * torch.randn(C, K, generator=g_)).to(bf),
             A_log=torch.log(torch.logspace(-2.7, 0.3, Hv)), dt=torch.zeros(Hv),
             nw=(1 + 0.02 * torch.randn(D, generator=g_)).to(bf),
             s0=0.02 * torch.randn(len(lens), Hv, D, D, generator=g_),
             hist=torch.randn(len(lens), C, K, generator=g_).to(bf))
    ref_core, ref_conv, ref_rec = oracle.gdn_prefill_core(x["mixed"], x["z"], x["a"], x["b"], x["cw"], x["A_log"],
                                                          x["dt"], x["nw"], Hk, Hv, D, cu_seqlens=cu,
                                                          conv_history=x["hist"], initial_state=x["s0"])
    d = {k: v.to(dev) for k, v in x.items()}
    core, conv, rec = gdn.gdn_prefill_core(d["mixed"], d["z"], d["a"], d["b"], d["cw"], d["A_log"], d["dt"], d["nw"],
                                           Hk, Hv, D, cu_seqlens=cu, conv_history=d["hist"], initial_state=d["s0"])
    torch.cuda.synchronize()
    assert torch.equal(conv.cpu(), ref_conv)
    for s_ in range(len(lens)):
        lo, hi = int(cu[s_]), int(cu[s_ + 1])
        assert rel_l2(core[lo:hi], ref_core[lo:hi]) <= OUT_TOL, f"prompt {s_}"
        for h in range(Hv):
            e = rel_l2(rec[s_, h], ref_rec[s_, h])
            assert e <= STATE_TOL, (s_, h, e)


@pytest.mark.gpu
def test_long_sequence_T32768_full_width(gdn, oracle, dev):
    """B=1, T=32768, H_k=16 read by H_v=32 value heads; q, k ~ N(0,1) (l2-normalised in the kernel),
    v ~ N(0,1), beta = sigmoid(N(0,1)), g = -0.1 softplus(N(0,1) + 2), S0 ~ N(0, 0.02), seed 3.
    The whole width runs on the GPU, and every value head is checked against the oracle."""
    T = 32768
    g_ = torch.Generator().manual_seed(3)
    bf = torch.bfloat16
    q = torch.randn(1, T, HK, D, generator=g_).to(bf)
    k = torch.randn(1, T, HK, D, generator=g_).to(bf)
    v = torch.randn(1, T, HV, D, generator=g_).to(bf)
    beta = torch.sigmoid(torch.randn(1, T, HV, generator=g_)).to(bf)
    g = -torch.nn.functional.softplus(torch.randn(1, T, HV, generator=g_) + 2) * 0.1
    s0 = 0.02 * torch.randn(1, HV, D, D, generator=g_)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    heads = list(range(HV))
    kh = [h // (HV // HK) for h in heads]
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q[:, :, kh], k[:, :, kh], v[:, :, heads], g[:, :, heads],
                                                    beta[:, :, heads], 64, s0[:, heads], True, True)
    assert rel_l2(o[:, :, heads], o_ref) <= OUT_TOL
    assert rel_l2(s[:, heads], s_ref) <= STATE_TOL
    for i, h in enumerate(heads):
        assert rel_l2(s[:, h], s_ref[:, i]) <= STATE_TOL, f"value head {h}"


@pytest.mark.gpu
def test_T8192_model_shape_Hv48(gdn, oracle, dev):
    """The chunked rule at Qwen3.5-27B's GDN shape (H_k=16 key heads read by H_v=48 value heads,
    src/cb_tp.py:7-10) at T=8192: 5 segments of 26 chunks per value head, 240 (segment, value head)
    items.  Seven value heads spread over the key heads (all three of key head 0) against the oracle."""
    T, Hk, Hv = 8192, 16, 48
    g_ = torch.Generator().manual_seed(48)
    bf = torch.bfloat16
    q = torch.randn(1, T, Hk, D, generator=g_).to(bf)
    k = torch.randn(1, T, Hk, D, generator=g_).to(bf)
    v = torch.randn(1, T, Hv, D, generator=g_).to(bf)
    beta = torch.sigmoid(torch.randn(1, T, Hv, generator=g_)).to(bf)
    g = -torch.nn.functional.softplus(torch.randn(1, T, Hv, generator=g_) + 2) * 0.1
    s0 = 0.02 * torch.randn(1, Hv, D, D, generator=g_)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    heads = [0, 1, 2, 23, 24, 40, 47]
    kh = [h // (Hv // Hk) for h in heads]
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q[:, :, kh], k[:, :, kh], v[:, :, heads], g[:, :, heads],
                                                    beta[:, :, heads], 64, s0[:, heads], True, True)
    for i, h in enumerate(heads):
        assert rel_l2(o[:, :, h], o_ref[:, :, i]) <= OUT_TOL, f"value head {h}"
        assert rel_l2(s[:, h], s_ref[:, i]) <= STATE_TOL, f"value head {h}"


def _hybrid():
    from importlib import import_module
    return import_module(PKG_NAME + ".hybrid_decode")


def _contexts(seed=4):
    g_ = torch.Generator().manual_seed(seed)
    return torch.randint(512, 4097, (16,), generator=g_)


@pytest.mark.gpu
def test_27b_shape_graph_replay_matches_eager(gdn, dev):
    """The whole 64-layer step at Qwen3.5-27B shape: three graph replays give the eager steps' logits
    and every GDN layer's states (conv bit for bit)."""
    hd = _hybrid()
    cfg = hd.HybridConfig()
    ctx = _contexts()
    eager = hd.HybridDecoder(cfg, 16, ctx, 8, dev, seed=7)
    graphed = hd.HybridDecoder(cfg, 16, ctx, 8, dev, seed=7)
    g_ = torch.Generator().manual_seed(8)
    inp = torch.randn(16, cfg.hidden, generator=g_).to(torch.bfloat16).to(dev)
    graph = hd.HybridDecodeGraph(graphed, inp)        # one eager warm-up step inside
    eager.step(inp)
    for _ in range(3):
        out_g = graph.replay().clone()
        out_e = eager.step(inp)
        torch.cuda.synchronize()
        assert rel_l2(out_g, out_e) <= 1e-3
        for i in eager.slots.rec:
            assert torch.equal(graphed.slots.conv[i], eager.slots.conv[i])
            assert rel_l2(graphed.slots.rec[i], eager.slots.rec[i]) <= 1e-5
        assert torch.equal(graphed.pos, eager.pos)
    del eager, graphed, graph
    torch.cuda.empty_cache()


@pytest.mark.gpu
def test_27b_shape_gdn_layer_vs_oracle(gdn, oracle, dev):
    """One GDN layer at 27B shape (hidden 5120, H_k=16, H_v=48, conv 10240 x 4), 16 slots: the
    in-projection GEMM, the fused HIP core and out_proj against the oracle's decode core fed the same
    projections, and the layer's states after the step."""
    hd = _hybrid()
    cfg = hd.HybridConfig(layers=4)                   # the 27B layer shapes; layer 0 is a GDN layer
    model = hd.HybridDecoder(cfg, 16, _contexts(), 4, dev, seed=9, keep_plain=True)
    L = model.layers[0]
    g_ = torch.Generator().manual_seed(10)
    x = torch.randn(16, cfg.hidden, generator=g_).to(torch.bfloat16)
    with torch.no_grad():                              # random non-zero slot states
        model.slots.conv[0].copy_(torch.randn(model.slots.conv[0].shape, generator=g_).to(torch.bfloat16))
        model.slots.rec[0].copy_(0.02 * torch.randn(model.slots.rec[0].shape, generator=g_))
    conv0, rec0 = model.slots.conv[0].cpu(), model.slots.rec[0].cpu()
    # the projection the layer forms (its packed-weight HIP product, deterministic), checked against an
    # fp32 GEMM, then fed to the oracle: the conv state (the pre-conv inputs shifted in) is exact
    cb = importlib.import_module(PKG_NAME + ".cb_engine")
    proj = cb.decode_linear(x.to(dev), L.in_proj_p).cpu()
    assert rel_l2(proj, x.float() @ L.in_proj.cpu().float().t()) <= 1e-2
    out = model.gdn(0, L, x.to(dev)).cpu()
    Hk, Hv, Dh, Cc = cfg.gdn_k_heads, cfg.gdn_v_heads, cfg.gdn_head, cfg.conv_dim
    mixed, z = proj[:, :Cc], proj[:, Cc:Cc + Hv * Dh]
    b, a = proj[:, Cc + Hv * Dh:Cc + Hv * Dh + Hv], proj[:, Cc + Hv * Dh + Hv:]
    conv_ref, rec_ref = conv0.clone(), rec0.clone()
    core = oracle.gdn_decode_core(mixed, z, a, b, conv_ref, L.conv_w.cpu(), L.A_log.cpu(), L.dt_bias.cpu(),
                                  L.norm_w.cpu(), rec_ref, Hk, Hv, Dh, cfg.eps)
    ref = core.float() @ L.out.cpu().float().t()
    assert rel_l2(out, ref) <= OUT_TOL
    assert rel_l2(model.slots.rec[0], rec_ref) <= STATE_TOL
    assert torch.equal(model.slots.conv[0].cpu(), conv_ref)
