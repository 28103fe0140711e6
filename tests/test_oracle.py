"""CPU pins of the oracle (no GPU): each oracle function is checked against the transformers
routine the reference patches (installed transformers; the reference pins 5.5.4, these bodies are
unchanged in the installed version), against library routines and closed forms, and against
invariances of the recurrence.  The planted-mistake tests at the end mutate the oracle and confirm
that these pins catch a dropped term, a wrong sign and a transposed operand.
"""
import importlib

import pytest
import torch
import torch.nn.functional as F

from conftest import rel_l2

HF = importlib.import_module("transformers.models.qwen3_5.modeling_qwen3_5")


def config0(seed=0, T=512, H=4, d=64):
    """Config 0: B=1, T=512, H=4, d=64, fp32; q,k ~N(0,1) l2-normalised per head, v ~N(0,1),
    beta = sigmoid(N(0,1)), g = -softplus(N(0,1)+2)*0.1, zero initial state, chunk 64, seed 0."""
    g_ = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(1, T, H, d, generator=g_), dim=-1)
    k = F.normalize(torch.randn(1, T, H, d, generator=g_), dim=-1)
    v = torch.randn(1, T, H, d, generator=g_)
    beta = torch.sigmoid(torch.randn(1, T, H, generator=g_))
    g = -F.softplus(torch.randn(1, T, H, generator=g_) + 2) * 0.1
    return q, k, v, g, beta


# ---------------------------------------------------------------- l2norm
def test_l2norm_matches_hf_on_vectorised_shapes(oracle):
    x = torch.randn(1, 64, 4, 128).to(torch.bfloat16)          # 256 rows: no scalar tail in torch
    assert torch.equal(oracle.l2norm(x), HF.l2norm(x))
    xf = torch.randn(3, 5, 7, 64)
    assert torch.equal(oracle.l2norm(xf), HF.l2norm(xf))        # fp32: identical ops


def test_l2norm_within_one_ulp_of_hf_anywhere(oracle):
    x = torch.randn(1, 150, 2, 128).to(torch.bfloat16)          # 300 rows: torch double-rounds its tail
    a, b = oracle.l2norm(x).float(), HF.l2norm(x).float()
    assert ((a - b).abs() <= b.abs() * 2 ** -6 + 1e-12).all()   # 1 ulp of the inverse norm + rounding


# ---------------------------------------------------------------- inverse
def test_unit_lower_inv_is_the_inverse(oracle):
    g_ = torch.Generator().manual_seed(1)
    X = (torch.randn(8, 64, 64, generator=g_) * 0.3).tril(-1)
    T = oracle.unit_lower_inv(X)
    I = torch.eye(64)
    assert (T @ (I - X) - I).abs().max() < 1e-4
    exact = torch.linalg.solve_triangular((I - X).double(), I.double().expand(8, 64, 64), upper=False)
    assert rel_l2(T, exact) < 1e-6
    assert rel_l2(oracle.small_unit_lower_inv(X[:, :16, :16]), exact[:, :16, :16]) < 1e-6


# ---------------------------------------------------------------- chunked rule
def test_config0_chunked_equals_token_recurrence(oracle):
    q, k, v, g, beta = config0()
    o_c, s_c = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, None, True, False)
    o_r, s_r = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, None, True, False)
    assert rel_l2(o_c, o_r) < 1e-5 and rel_l2(s_c, s_r) < 1e-5


def test_positive_g_head_chunked_equals_token_recurrence(oracle):
    """The reference's decay exp((G_i - G_j).tril()) (src/gdn_chunk_fast2.py:41) holds for any sign of g;
    with one head growing (g > 0) the chunked rule still equals the token recurrence."""
    q, k, v, g, beta = config0(seed=5)
    g[..., 1] = -g[..., 1] * 0.02          # head 1: g in (0, 0.01], the state grows
    o_c, s_c = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, None, True, False)
    o_r, s_r = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, None, True, False)
    assert rel_l2(o_c, o_r) < 1e-5 and rel_l2(s_c, s_r) < 1e-5
    assert s_r[:, 1].norm() > s_r[:, 0].norm()


def test_chunked_matches_hf_chunk_and_recurrent(oracle):
    q, k, v, g, beta = config0(seed=3, T=200)
    s0 = 0.02 * torch.randn(1, 4, 64, 64)
    o, s = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, s0, True, True)
    o_hf, s_hf = HF.torch_chunk_gated_delta_rule(q, k, v, g, beta, 64, s0, True, True)
    o_tr, s_tr = HF.torch_recurrent_gated_delta_rule(q, k, v, g, beta, s0, True, True)
    assert rel_l2(o, o_hf) < 1e-5 and rel_l2(s, s_hf) < 1e-5
    assert rel_l2(o, o_tr) < 1e-5 and rel_l2(s, s_tr) < 1e-5
    o1, s1 = oracle.chunk_gated_delta_rule_v1(q, k, v, g, beta, 64, s0, True, True)
    assert rel_l2(o1, o) < 1e-6 and rel_l2(s1, s) < 1e-6


def test_chunked_bf16_inputs_match_hf(oracle):
    g_ = torch.Generator().manual_seed(4)
    q = torch.randn(1, 128, 2, 128, generator=g_).to(torch.bfloat16)   # 256 rows
    k = torch.randn(1, 128, 2, 128, generator=g_).to(torch.bfloat16)
    v = torch.randn(1, 128, 2, 128, generator=g_).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(1, 128, 2, generator=g_)).to(torch.bfloat16)
    g = -torch.rand(1, 128, 2, generator=g_) * 0.5
    o, s = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, None, True, True)
    o_hf, s_hf = HF.torch_chunk_gated_delta_rule(q, k, v, g, beta, 64, None, True, True)
    assert o.dtype == torch.bfloat16
    assert rel_l2(o, o_hf) < 1e-2 and rel_l2(s, s_hf) < 1e-5


def test_padding_and_split_invariance(oracle):
    q, k, v, g, beta = config0(seed=5, T=300)
    o, s = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, None, True)
    o_a, s_a = oracle.chunk_gated_delta_rule_v2(q[:, :100], k[:, :100], v[:, :100], g[:, :100],
                                                beta[:, :100], 64, None, True)
    o_b, s_b = oracle.chunk_gated_delta_rule_v2(q[:, 100:], k[:, 100:], v[:, 100:], g[:, 100:],
                                                beta[:, 100:], 64, s_a, True)
    assert rel_l2(torch.cat([o_a, o_b], 1), o) < 1e-5 and rel_l2(s_b, s) < 1e-5


def test_varlen_equals_independent_calls(oracle):
    q, k, v, g, beta = config0(seed=6, T=230)
    cu = torch.tensor([0, 70, 70, 200, 230])
    s0 = 0.02 * torch.randn(4, 4, 64, 64)
    o, s = oracle.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu, 64, s0, True)
    for i in range(4):
        a, b = int(cu[i]), int(cu[i + 1])
        oi, si = HF.torch_recurrent_gated_delta_rule(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b],
                                                     beta[:, a:b], s0[i:i + 1], True)
        assert rel_l2(s[i:i + 1], si) < 1e-5
        if b > a:
            assert rel_l2(o[:, a:b], oi) < 1e-5


# ---------------------------------------------------------------- decode step
def test_recurrent_single_step_bit_exact_vs_hf(oracle):
    g_ = torch.Generator().manual_seed(7)
    N, H, D = 16, 4, 128                                           # 64 rows: vectorised l2norm
    q = torch.randn(N, 1, H, D, generator=g_).to(torch.bfloat16)
    k = torch.randn(N, 1, H, D, generator=g_).to(torch.bfloat16)
    v = torch.randn(N, 1, H, D, generator=g_).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(N, 1, H, generator=g_)).to(torch.bfloat16)
    g = -torch.rand(N, 1, H, generator=g_)
    S = 0.02 * torch.randn(N, H, D, D, generator=g_)
    o, s = oracle.recurrent_single_step(q, k, v, g, beta, S, True, True)
    o_hf, s_hf = HF.torch_recurrent_gated_delta_rule(q, k, v, g, beta, S, True, True)
    assert torch.equal(o, o_hf) and torch.equal(s, s_hf)


def test_recurrent_single_step_special_cases(oracle):
    g_ = torch.Generator().manual_seed(8)
    N, H, D = 2, 3, 32
    q = F.normalize(torch.randn(N, 1, H, D, generator=g_), dim=-1)
    v = torch.randn(N, 1, H, D, generator=g_)
    g = -torch.rand(N, 1, H, generator=g_)
    S = torch.randn(N, H, D, D, generator=g_)
    # beta = 0: pure decay, o = e^g S^T q d^-1/2
    k = F.normalize(torch.randn(N, 1, H, D, generator=g_), dim=-1)
    o, s = oracle.recurrent_single_step(q, k, v, g, torch.zeros(N, 1, H), S, True)
    gam = g[:, 0].exp()[..., None, None]
    assert torch.allclose(s, S * gam, atol=1e-6)
    assert torch.allclose(o[:, 0], torch.einsum("nhkv,nhk->nhv", S * gam, q[:, 0]) / D ** 0.5, atol=1e-5)
    # zero state: o = beta (k.q) v d^-1/2, S' = beta k v^T
    beta = torch.rand(N, 1, H, generator=g_)
    o, s = oracle.recurrent_single_step(q, k, v, g, beta, None, True)
    kq = (k[:, 0] * q[:, 0]).sum(-1, keepdim=True) / D ** 0.5
    assert torch.allclose(o[:, 0], beta[:, 0, :, None] * kq * v[:, 0], atol=1e-6)
    # exact write: g = 0, beta = 1, unit k -> S'^T k = v
    o, s = oracle.recurrent_single_step(q, k, v, torch.zeros(N, 1, H), torch.ones(N, 1, H), S, True)
    assert torch.allclose(torch.einsum("nhkv,nhk->nhv", s, k[:, 0]), v[:, 0], atol=1e-4)


# ---------------------------------------------------------------- conv
def test_elem_conv_update_integer_kat_and_hf(oracle):
    N, C, K = 2, 16, 4
    x = torch.arange(N * C).reshape(N, C, 1).remainder(5).sub(2).to(torch.bfloat16)
    st = torch.arange(N * C * K).reshape(N, C, K).remainder(7).sub(3).to(torch.bfloat16)
    w = torch.arange(C * K).reshape(C, K).remainder(3).sub(1).to(torch.bfloat16)
    st1 = st.clone()
    out = oracle.elem_conv_update(x, st1, w, None)
    win = torch.cat([st[:, :, 1:], x], -1)
    dot = sum(win[:, :, i].float() * w[:, i].float() for i in range(K))    # exact small integers
    assert torch.equal(st1, win)
    assert torch.equal(out[:, :, 0], (dot * torch.sigmoid(dot)).to(torch.bfloat16))
    g_ = torch.Generator().manual_seed(9)
    x = torch.randn(4, 64, 1, generator=g_).to(torch.bfloat16)
    st = torch.randn(4, 64, K, generator=g_).to(torch.bfloat16)
    w = torch.randn(64, K, generator=g_).to(torch.bfloat16)
    s_a, s_b = st.clone(), st.clone()
    a = oracle.elem_conv_update(x, s_a, w, None)
    b = HF.causal_conv1d_update(x, s_b, w, None, "silu")
    assert torch.equal(s_a, s_b)
    assert ((a.float() - b.float()).abs() <= b.float().abs() * 2 ** -5 + 2 ** -6).all()


def test_conv_prefill_equals_repeated_updates(oracle):
    g_ = torch.Generator().manual_seed(10)
    C, K, L = 32, 4, 9
    x = torch.randn(1, C, L, generator=g_).to(torch.bfloat16)
    w = torch.randn(C, K, generator=g_).to(torch.bfloat16)
    for hist in (None, torch.randn(1, C, K, generator=g_).to(torch.bfloat16)):
        out, st = oracle.causal_conv1d_prefill(x, w, None, hist)
        s = torch.zeros(1, C, K, dtype=torch.bfloat16) if hist is None else hist.clone()
        outs = [oracle.causal_conv1d_update(x[:, :, t:t + 1], s, w, None, "silu") for t in range(L)]
        assert torch.equal(st, s), "prefill leaves the state L decode updates leave"
        ref = torch.cat(outs, -1)
        assert ((out.float() - ref.float()).abs() <= ref.float().abs() * 2 ** -7 + 1e-6).all()
    _, st_short = oracle.causal_conv1d_prefill(x[:, :, :2], w, None, None)
    assert torch.equal(st_short[:, :, :2], torch.zeros(1, C, 2, dtype=torch.bfloat16))
    assert torch.equal(st_short[:, :, 2:], x[:, :, :2])


# ---------------------------------------------------------------- gated norm, gating
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_gated_rmsnorm_bit_exact_vs_hf_module(oracle, wdtype):
    g_ = torch.Generator().manual_seed(11)
    x = torch.randn(64, 128, generator=g_).to(torch.bfloat16)
    z = torch.randn(64, 128, generator=g_).to(torch.bfloat16)
    mod = HF.Qwen3_5RMSNormGated(128, eps=1e-6)
    with torch.no_grad():
        mod.weight.copy_(1 + 0.02 * torch.randn(128, generator=g_))
    mod = mod.to(wdtype)
    with torch.no_grad():
        ref = mod(x, z)
    assert torch.equal(oracle.gated_rmsnorm(x, z, mod.weight.detach(), 1e-6), ref)


def test_gating_closed_form(oracle):
    g_ = torch.Generator().manual_seed(12)
    a = torch.randn(64, 32, generator=g_).to(torch.bfloat16)
    b = torch.randn(64, 32, generator=g_).to(torch.bfloat16)
    A_log = torch.log(torch.rand(32, generator=g_) * 16 + 0.01)
    dt = torch.rand(32, generator=g_)
    beta, g = oracle.gdn_gating(a, b, A_log, dt)
    ad = a.double() + dt.double()
    g64 = -A_log.double().exp() * torch.where(ad > 20, ad, torch.log1p(ad.exp()))
    assert rel_l2(g, g64) < 1e-6
    assert torch.equal(beta, torch.sigmoid(b.double()).to(torch.bfloat16))


# ---------------------------------------------------------------- layer compositions
def test_prefill_then_decode_equals_longer_prefill(oracle):
    """Prefill T tokens, then one decode step, equals prefill of T+1 tokens (state carried by the
    slot layout: conv state = last K pre-conv inputs, recurrent state fp32)."""
    Hk, Hv, D, K, T = 1, 2, 32, 4, 70
    C = (2 * Hk + Hv) * D
    g_ = torch.Generator().manual_seed(13)
    mixed = torch.randn(T + 1, C, generator=g_).to(torch.bfloat16)
    z = torch.randn(T + 1, Hv * D, generator=g_).to(torch.bfloat16)
    a = torch.randn(T + 1, Hv, generator=g_).to(torch.bfloat16)
    b = torch.randn(T + 1, Hv, generator=g_).to(torch.bfloat16)
    cw = (0.5 * torch.randn(C, K, generator=g_)).to(torch.bfloat16)
    A_log, dt = torch.full((Hv,), -2.3), torch.full((Hv,), 2.0)
    nw = torch.ones(D).to(torch.bfloat16)
    core_all, conv_all, rec_all = oracle.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D)
    _, conv_t, rec_t = oracle.gdn_prefill_core(mixed[:T], z[:T], a[:T], b[:T], cw, A_log, dt, nw, Hk, Hv, D)
    last = oracle.gdn_decode_core(mixed[T:], z[T:], a[T:], b[T:], conv_t, cw, A_log, dt, nw, rec_t, Hk, Hv, D)
    assert torch.equal(conv_t, conv_all)
    assert rel_l2(rec_t, rec_all) < 1e-2        # conv rounding differs between prefill and decode
    assert rel_l2(last, core_all[T:]) < 5e-2


# ---------------------------------------------------------------- planted mistakes
def _mutants(oracle):
    """Oracle chunked rules with one plausible mistake each."""
    def dropped_decay(q, k, v, g, beta, *a, **kw):     # decay term dropped
        return oracle.chunk_gated_delta_rule_v2(q, k, v, torch.zeros_like(g), beta, *a, **kw)

    def wrong_sign(q, k, v, g, beta, *a, **kw):        # X sign flipped: (I + X)^-1 instead of (I - X)^-1
        orig = oracle.unit_lower_inv
        oracle.unit_lower_inv = lambda X, base=16: orig(-X, base)
        try:
            return oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, *a, **kw)
        finally:
            oracle.unit_lower_inv = orig

    def transposed(q, k, v, g, beta, *a, **kw):        # q and k swapped
        return oracle.chunk_gated_delta_rule_v2(k, q, v, g, beta, *a, **kw)

    def no_beta_on_v(q, k, v, g, beta, *a, **kw):      # beta dropped from the value write
        return oracle.chunk_gated_delta_rule_v2(q, k, v / beta.unsqueeze(-1).clamp_min(1e-3), g, beta, *a, **kw)

    return {"dropped_decay": dropped_decay, "wrong_sign": wrong_sign, "transposed": transposed,
            "no_beta_on_v": no_beta_on_v}


@pytest.mark.parametrize("name", ["dropped_decay", "wrong_sign", "transposed", "no_beta_on_v"])
def test_planted_mistake_is_caught_by_token_recurrence_pin(oracle, name):
    q, k, v, g, beta = config0(seed=14, T=130)
    fn = _mutants(oracle)[name]
    o_m, s_m = fn(q, k, v, g, beta, 64, None, True)
    o_r, s_r = HF.torch_recurrent_gated_delta_rule(q, k, v, g, beta, None, True)
    assert rel_l2(o_m, o_r) > 1e-2 or rel_l2(s_m, s_r) > 1e-2, f"pin missed mutant {name}"
