"""GPU parity of the decode kernels against the CPU oracle (same seeded inputs).

Tolerances (from the path's contract): output rel-L2 <= 1e-2 (bf16 activations), fp32 recurrent
state rel-L2 <= 1e-3, conv-state shifting and slot indexing bit-exact.
"""
import pytest
import torch

from conftest import assert_same_bits, normal_bf16_values, rel_l2

pytestmark = pytest.mark.gpu

OUT_TOL = 1e-2
STATE_TOL = 1e-3


def _decode_inputs(N, Hk, Hv, D, seed=0, dtype=torch.bfloat16, state_std=0.02):
    g_ = torch.Generator().manual_seed(seed)
    q = torch.randn(N, 1, Hk, D, generator=g_).to(dtype)
    k = torch.randn(N, 1, Hk, D, generator=g_).to(dtype)
    v = torch.randn(N, 1, Hv, D, generator=g_).to(dtype)
    beta = torch.sigmoid(torch.randn(N, 1, Hv, generator=g_)).to(dtype)
    g = -torch.nn.functional.softplus(torch.randn(N, 1, Hv, generator=g_) + 2) * 0.1
    S = torch.randn(N, Hv, D, D, generator=g_) * state_std
    return q, k, v, g, beta, S


@pytest.mark.parametrize("l2", [True, False])
@pytest.mark.parametrize("repeat", [True, False])
def test_recurrent_single_step_bf16(gdn, oracle, dev, l2, repeat):
    N, Hk, Hv, D = 16, 16, 32, 128
    q, k, v, g, beta, S = _decode_inputs(N, Hk, Hv, D, seed=1)
    if repeat:  # the engine's repeat_interleave'd layout
        q, k = q.repeat_interleave(2, dim=2), k.repeat_interleave(2, dim=2)
    o_ref, s_ref = oracle.recurrent_single_step(q.repeat_interleave(2, 2) if not repeat else q,
                                                k.repeat_interleave(2, 2) if not repeat else k,
                                                v, g, beta, S, True, l2)
    S_dev = S.to(dev)
    S_keep = S_dev.clone()
    o, s = gdn.recurrent_single_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), S_dev,
                                     True, l2)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and o.shape == (N, 1, Hv, D)
    assert torch.equal(S_dev, S_keep), "input state must not be mutated (out-of-place contract)"
    assert rel_l2(o, o_ref) <= OUT_TOL
    assert rel_l2(s, s_ref) <= STATE_TOL


def test_recurrent_single_step_inplace_and_none_state(gdn, oracle, dev):
    N, H, D = 4, 8, 128
    q, k, v, g, beta, S = _decode_inputs(N, H, H, D, seed=2)
    o_ref, s_ref = oracle.recurrent_single_step(q, k, v, g, beta, S, True, True)
    S_dev = S.to(dev)
    o, s = gdn.recurrent_single_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), S_dev,
                                     True, True, inplace=True)
    assert s.data_ptr() == S_dev.data_ptr()
    assert rel_l2(S_dev, s_ref) <= STATE_TOL and rel_l2(o, o_ref) <= OUT_TOL
    # zero initial state (None): o = beta * (k.q) * v
    o0_ref, s0_ref = oracle.recurrent_single_step(q, k, v, g, beta, None, True, True)
    o0, s0 = gdn.recurrent_single_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), None,
                                       True, True)
    assert rel_l2(o0, o0_ref) <= OUT_TOL and rel_l2(s0, s0_ref) <= STATE_TOL
    _, none_state = gdn.recurrent_single_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              None, False, True)
    assert none_state is None


def test_recurrent_single_step_fp32_and_multi_token(gdn, oracle, dev):
    N, H, D, T = 2, 4, 128, 5
    g_ = torch.Generator().manual_seed(3)
    q = torch.randn(N, T, H, D, generator=g_)
    k = torch.randn(N, T, H, D, generator=g_)
    v = torch.randn(N, T, H, D, generator=g_)
    beta = torch.sigmoid(torch.randn(N, T, H, generator=g_))
    g = -torch.rand(N, T, H, generator=g_) * 0.5
    S = torch.randn(N, H, D, D, generator=g_) * 0.02
    o_ref, s_ref = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, S, True, True)
    o, s = gdn.recurrent_single_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), S.to(dev),
                                     True, True)
    assert o.dtype == torch.float32
    assert rel_l2(o, o_ref) <= 1e-5 and rel_l2(s, s_ref) <= 1e-5


def test_elem_conv_update_bit_exact_state(gdn, oracle, dev):
    N, C, K = 16, 8192, 4
    g_ = torch.Generator().manual_seed(4)
    x = torch.randn(N, C, 1, generator=g_).to(torch.bfloat16)
    st = torch.randn(N, C, K, generator=g_).to(torch.bfloat16)
    w = torch.randn(C, K, generator=g_).to(torch.bfloat16)
    bias = torch.randn(C, generator=g_).to(torch.bfloat16)
    for b in (None, bias):
        st_ref = st.clone()
        o_ref = oracle.elem_conv_update(x, st_ref, w, b)
        st_dev = st.to(dev)
        o = gdn.elem_conv_update(x.to(dev), st_dev, w.to(dev), None if b is None else b.to(dev))
        assert torch.equal(st_dev.cpu(), st_ref), "conv state shift must be bit-exact"
        diff = (o.cpu().float() - o_ref.float()).abs()
        ulp = o_ref.float().abs().clamp_min(2 ** -126) * 2 ** -7
        assert (diff <= ulp).all(), "conv output off by more than one bf16 ulp"
        assert (diff == 0).float().mean().item() >= 0.999


def test_elem_conv_update_silu_every_bf16_input(gdn, oracle, dev):
    """The decode conv's SiLU is torch's, bit for bit, for every normal bf16 input (taps (0, 0, 0, 1)
    and a zero state: the conv value is the input)."""
    x = normal_bf16_values()
    x = torch.cat([x, torch.zeros(-x.numel() % 8, dtype=x.dtype)])  # whole 8-channel groups
    C, K = x.numel(), 4
    w = torch.zeros(C, K, dtype=torch.bfloat16)
    w[:, K - 1] = 1
    st = torch.zeros(1, C, K, dtype=torch.bfloat16)
    o_ref = oracle.elem_conv_update(x.reshape(1, C, 1), st.clone(), w, None)
    o = gdn.elem_conv_update(x.reshape(1, C, 1).to(dev), st.to(dev), w.to(dev), None)
    assert_same_bits(o, o_ref, x)


def test_elem_conv_update_integer_kat(gdn, dev):
    """Integer-valued bf16 inputs: every product and sum is exact, so out = silu(dot) exactly."""
    N, C, K = 3, 64, 4
    x = torch.arange(N * C).reshape(N, C, 1).remainder(7).sub(3).to(torch.bfloat16)
    st = torch.arange(N * C * K).reshape(N, C, K).remainder(5).sub(2).to(torch.bfloat16)
    w = torch.arange(C * K).reshape(C, K).remainder(3).sub(1).to(torch.bfloat16)
    win = torch.cat([st[:, :, 1:], x], dim=-1)
    dot = (win.float() * w.float()).sum(-1, keepdim=True)
    expect = torch.nn.functional.silu(dot.to(torch.bfloat16).float()).to(torch.bfloat16)
    st_dev = st.to(dev)
    o = gdn.elem_conv_update(x.to(dev), st_dev, w.to(dev), None)
    assert torch.equal(st_dev.cpu(), win)
    assert torch.equal(o.cpu(), expect)


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_gated_rmsnorm(gdn, oracle, dev, wdtype):
    rows, D = 16 * 32, 128
    g_ = torch.Generator().manual_seed(5)
    x = torch.randn(rows, D, generator=g_).to(torch.bfloat16)
    z = torch.randn(rows, D, generator=g_).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(D, generator=g_)).to(wdtype)
    ref = oracle.gated_rmsnorm(x, z, w, 1e-6)
    out = gdn.gated_rmsnorm(x.to(dev), z.to(dev), w.to(dev), 1e-6)
    diff = (out.cpu().float() - ref.float()).abs()
    assert (diff <= ref.float().abs() * 2 ** -7 + 1e-30).all()
    assert (diff == 0).float().mean().item() >= 0.99


def _layer_inputs(N, Hk, Hv, D, K, seed):
    g_ = torch.Generator().manual_seed(seed)
    C = (2 * Hk + Hv) * D
    p = dict(
        mixed=torch.randn(N, C, generator=g_).to(torch.bfloat16),
        z=torch.randn(N, Hv * D, generator=g_).to(torch.bfloat16),
        a=torch.randn(N, Hv, generator=g_).to(torch.bfloat16),
        b=torch.randn(N, Hv, generator=g_).to(torch.bfloat16),
        conv_state=torch.randn(N, C, K, generator=g_).to(torch.bfloat16),
        conv_weight=(torch.randn(C, K, generator=g_) * 0.5).to(torch.bfloat16),
        A_log=torch.full((Hv,), float(torch.log(torch.tensor(0.1)))),
        dt_bias=torch.full((Hv,), 2.0),
        norm_weight=(1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16),
        rec_state=torch.randn(N, Hv, D, D, generator=g_) * 0.02,
    )
    return p


@pytest.mark.parametrize("Hk,Hv", [(16, 32), (16, 48), (8, 8), (4, 16)])
def test_decode_fused_layer(gdn, oracle, dev, Hk, Hv):
    N, D, K = 16, 128, 4
    p = _layer_inputs(N, Hk, Hv, D, K, seed=6)
    ref_conv, ref_rec = p["conv_state"].clone(), p["rec_state"].clone()
    ref = oracle.gdn_decode_core(p["mixed"], p["z"], p["a"], p["b"], ref_conv, p["conv_weight"],
                                 p["A_log"], p["dt_bias"], p["norm_weight"], ref_rec, Hk, Hv, D)
    d = {k: v.to(dev) for k, v in p.items()}
    out = gdn.gdn_decode_core(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_weight"],
                              d["A_log"], d["dt_bias"], d["norm_weight"], d["rec_state"], Hk, Hv, D)
    torch.cuda.synchronize()
    assert torch.equal(d["conv_state"].cpu(), ref_conv), "conv state must be bit-exact"
    assert rel_l2(out, ref) <= OUT_TOL
    assert rel_l2(d["rec_state"], ref_rec) <= STATE_TOL


@pytest.mark.parametrize("Hk,Hv,K,wdtype", [(16, 48, 3, torch.float32), (4, 16, 2, torch.float32),
                                             (8, 8, 4, torch.float32)])
def test_decode_fused_layer_conv_k_and_fp32_norm(gdn, oracle, dev, Hk, Hv, K, wdtype):
    """Conv kernel sizes other than 4 (window updated in place in the prologue) and an fp32 norm weight."""
    N, D = 16, 128
    p = _layer_inputs(N, Hk, Hv, D, K, seed=8)
    p["norm_weight"] = p["norm_weight"].to(wdtype)
    ref_conv, ref_rec = p["conv_state"].clone(), p["rec_state"].clone()
    ref = oracle.gdn_decode_core(p["mixed"], p["z"], p["a"], p["b"], ref_conv, p["conv_weight"],
                                 p["A_log"], p["dt_bias"], p["norm_weight"], ref_rec, Hk, Hv, D)
    d = {k: v.to(dev) for k, v in p.items()}
    out = gdn.gdn_decode_core(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_weight"],
                              d["A_log"], d["dt_bias"], d["norm_weight"], d["rec_state"], Hk, Hv, D)
    torch.cuda.synchronize()
    assert torch.equal(d["conv_state"].cpu(), ref_conv), "conv state must be bit-exact"
    assert rel_l2(out, ref) <= OUT_TOL
    assert rel_l2(d["rec_state"], ref_rec) <= STATE_TOL


def test_decode_fused_slot_independence(gdn, dev):
    """Changing slot j's inputs leaves every other slot's output and state bit-identical."""
    N, Hk, Hv, D, K = 8, 4, 8, 128, 4
    p = _layer_inputs(N, Hk, Hv, D, K, seed=7)

    def run(pp):
        d = {k: v.to(dev) for k, v in pp.items()}
        out = gdn.gdn_decode_core(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_weight"],
                                  d["A_log"], d["dt_bias"], d["norm_weight"], d["rec_state"], Hk, Hv, D)
        return out.cpu(), d["conv_state"].cpu(), d["rec_state"].cpu()

    o1, c1, r1 = run(p)
    p2 = dict(p)
    j = 5
    for key in ("mixed", "z", "a", "b", "conv_state", "rec_state"):
        t = p[key].clone()
        t[j] = torch.randn_like(t[j].float()).to(t.dtype)
        p2[key] = t
    o2, c2, r2 = run(p2)
    keep = [i for i in range(N) if i != j]
    assert torch.equal(o1[keep], o2[keep]) and torch.equal(c1[keep], c2[keep]) and torch.equal(r1[keep], r2[keep])
    assert not torch.equal(o1[j], o2[j])


def test_decode_graph_replay_matches_eager(gdn, dev):
    """48-layer-style capture (3 layers here): every replay equals the eager step on the same state."""
    N, Hk, Hv, D, K, L = 16, 16, 32, 128, 4, 3
    layers = [_layer_inputs(N, Hk, Hv, D, K, seed=10 + i) for i in range(L)]
    dl = [{k: v.to(dev) for k, v in p.items()} for p in layers]
    eager = [{k: v.clone() for k, v in p.items()} for p in dl]

    def step(ls):
        outs = []
        for d in ls:
            outs.append(gdn.gdn_decode_core(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"],
                                            d["conv_weight"], d["A_log"], d["dt_bias"], d["norm_weight"],
                                            d["rec_state"], Hk, Hv, D))
        return torch.stack(outs)

    graph = gdn.GDNDecodeGraph(lambda: step(dl), device=dev)   # eager warm-up ran one step; capture runs none
    step(eager)
    for rep in range(3):
        out = graph.replay().clone()
        ref = step(eager)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from eager"
        for a, b in zip(dl, eager):
            assert torch.equal(a["rec_state"], b["rec_state"]) and torch.equal(a["conv_state"], b["conv_state"])
