"""GPU parity of the prefill kernels against the CPU oracle (same seeded inputs).

Tolerances: output rel-L2 <= 1e-2 (bf16 activations), final fp32 state rel-L2 <= 1e-3; conv state
capture bit-exact; the 64x64 inverse to fp32 rounding.
"""
import pytest
import torch

from conftest import assert_same_bits, normal_bf16_values, rel_l2

pytestmark = pytest.mark.gpu

OUT_TOL = 1e-2
STATE_TOL = 1e-3


def _gdn_inputs(T, Hk, Hv, D=128, seed=0, B=1, state=True, decay=0.1):
    g_ = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, Hk, D, generator=g_).to(torch.bfloat16)
    k = torch.randn(B, T, Hk, D, generator=g_).to(torch.bfloat16)
    v = torch.randn(B, T, Hv, D, generator=g_).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=g_)).to(torch.bfloat16)
    g = -torch.nn.functional.softplus(torch.randn(B, T, Hv, generator=g_) + 2) * decay
    s0 = 0.02 * torch.randn(B, Hv, D, D, generator=g_) if state else None
    return q, k, v, g, beta, s0


def _rep(x, r):
    return x.repeat_interleave(r, dim=2) if r > 1 else x


def test_unit_lower_inv(gdn, oracle, dev):
    """T (I - X) = I to fp32 rounding; equals the oracle's blocked inverse and solve_triangular."""
    g_ = torch.Generator().manual_seed(0)
    k = torch.nn.functional.normalize(torch.randn(64, 64, 128, generator=g_), dim=-1)
    beta = torch.rand(64, 64, generator=g_)
    G = torch.cumsum(-torch.rand(64, 64, generator=g_) * 0.3, dim=-1)
    dec = (G.unsqueeze(-1) - G.unsqueeze(-2)).tril().exp().tril()
    X = -((k * beta.unsqueeze(-1)) @ k.transpose(-1, -2) * dec).tril(-1)
    T = gdn._unit_lower_inv(X.to(dev)).cpu()
    I = torch.eye(64)
    exact = torch.linalg.solve_triangular((I - X).double(), I.double().expand(64, 64, 64), upper=False)
    assert rel_l2(T, exact) <= 1e-5
    assert rel_l2(T, oracle.unit_lower_inv(X)) <= 1e-5
    assert ((T.double() @ (I - X).double()) - I.double()).abs().max().item() <= 1e-4


@pytest.mark.parametrize("T,Hk,Hv,repeat", [(150, 2, 2, True), (1, 2, 4, False), (64, 2, 4, False),
                                            (65, 4, 8, False), (300, 16, 32, False), (129, 2, 6, False)])
def test_chunk_prefill_vs_oracle(gdn, oracle, dev, T, Hk, Hv, repeat):
    q, k, v, g, beta, s0 = _gdn_inputs(T, Hk, Hv, seed=T + Hv)
    r = Hv // Hk
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(_rep(q, r), _rep(k, r), v, g, beta, 64, s0, True, True)
    qd, kd = (_rep(q, r), _rep(k, r)) if repeat else (q, k)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(qd.to(dev), kd.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert o.shape == (1, T, Hv, 128) and o.dtype == torch.bfloat16
    assert rel_l2(o, o_ref) <= OUT_TOL, rel_l2(o, o_ref)
    assert rel_l2(s, s_ref) <= STATE_TOL, rel_l2(s, s_ref)


def test_chunk_prefill_v1_name_no_state_fp32_beta(gdn, oracle, dev):
    q, k, v, g, beta, _ = _gdn_inputs(200, 2, 2, seed=11, state=False)
    beta = beta.float()
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v1(q, k, v, g, beta, 64, None, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                           output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_l2(o, o_ref) <= OUT_TOL and rel_l2(s, s_ref) <= STATE_TOL
    _, none = gdn.fast_chunk_gated_delta_rule(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              use_qk_l2norm_in_kernel=True)
    assert none is None


def test_chunk_prefill_without_l2norm_and_batch(gdn, oracle, dev):
    """Pre-normalised q, k with use_qk_l2norm_in_kernel=False; B=3 dense batch."""
    q, k, v, g, beta, _ = _gdn_inputs(130, 2, 2, seed=12, B=3, state=False)
    q = oracle.l2norm(q)
    k = oracle.l2norm(k)
    s0 = 0.02 * torch.randn(3, 2, 128, 128)
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, s0, True, False)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True)
    assert rel_l2(o, o_ref) <= OUT_TOL and rel_l2(s, s_ref) <= STATE_TOL


def test_chunk_prefill_varlen_matches_per_sequence(gdn, oracle, dev):
    lens = [100, 64, 0, 236, 1, 65]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T = int(cu[-1])
    Hk, Hv = 4, 8
    q, k, v, g, beta, _ = _gdn_inputs(T, Hk, Hv, seed=13, state=False)
    s0 = 0.02 * torch.randn(len(lens), Hv, 128, 128)
    o_ref, s_ref = oracle.chunk_gated_delta_rule_varlen(_rep(q, 2), _rep(k, 2), v, g, beta, cu, 64, s0, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(dev))
    assert rel_l2(o, o_ref) <= OUT_TOL and rel_l2(s, s_ref) <= STATE_TOL
    assert torch.equal(s[2].cpu(), s0[2]), "an empty sequence keeps its initial state"
    with pytest.raises(ValueError):
        gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                           cu_seqlens=torch.tensor([0, 5, 3, T], dtype=torch.int32))


@pytest.mark.parametrize("with_state", [True, False])
def test_chunk_prefill_many_sequences_grouped(gdn, oracle, dev, with_state):
    """40 packed sequences at H_v=4: the scan streams several whole sequences per workgroup and
    carries the state across their boundaries (lengths 0, 1, 63, 64, 65 and random up to 200)."""
    g_ = torch.Generator().manual_seed(31)
    lens = [0, 1, 63, 64, 65, 0, 0, 130] + torch.randint(0, 201, (32,), generator=g_).tolist()
    lens[20] = 0
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T = int(cu[-1])
    Hk, Hv = 2, 4
    q, k, v, g, beta, _ = _gdn_inputs(T, Hk, Hv, seed=32, state=False)
    s0 = 0.02 * torch.randn(len(lens), Hv, 128, 128, generator=g_) if with_state else None
    o_ref, s_ref = oracle.chunk_gated_delta_rule_varlen(_rep(q, 2), _rep(k, 2), v, g, beta, cu, 64, s0, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev) if with_state else None,
                                              output_final_state=True, use_qk_l2norm_in_kernel=True,
                                              cu_seqlens=cu.tolist())
    assert rel_l2(o, o_ref) <= OUT_TOL
    for i, L in enumerate(lens):
        if L == 0:  # an empty sequence keeps its initial state exactly (zeros without one)
            assert torch.equal(s[i].cpu(), s0[i] if with_state else torch.zeros(Hv, 128, 128))
        else:
            assert rel_l2(s[i], s_ref[i]) <= STATE_TOL, (i, L)


def test_chunk_prefill_split_invariance(gdn, dev):
    """Prefill in two pieces with final -> initial state equals one call (prefill_chunk contract)."""
    q, k, v, g, beta, s0 = _gdn_inputs(320, 2, 4, seed=14)
    args = lambda a, b: [x[:, a:b].to(dev) for x in (q, k, v, g, beta)]
    o, s = gdn.fast_chunk_gated_delta_rule_v2(*args(0, 320), initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    o1, s1 = gdn.fast_chunk_gated_delta_rule_v2(*args(0, 128), initial_state=s0.to(dev), output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
    o2, s2 = gdn.fast_chunk_gated_delta_rule_v2(*args(128, 320), initial_state=s1, output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
    assert rel_l2(torch.cat([o1, o2], 1), o) <= 1e-3 and rel_l2(s2, s) <= 1e-5


def test_chunk_prefill_long_sequence_state_accuracy(gdn, oracle, dev):
    """T=32768 with 4 value heads (the long-sequence shape at reduced width): final-state rel-L2."""
    q, k, v, g, beta, s0 = _gdn_inputs(32768, 2, 4, seed=15)
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(_rep(q, 2), _rep(k, 2), v, g, beta, 64, s0, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    assert rel_l2(o, o_ref) <= OUT_TOL and rel_l2(s, s_ref) <= STATE_TOL


def test_chunk_prefill_slow_decay_state_accuracy(gdn, oracle, dev):
    """Slow decay (long memory across chunks) keeps the state within tolerance."""
    q, k, v, g, beta, s0 = _gdn_inputs(2048, 2, 2, seed=16, decay=0.005)
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, s0, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    assert rel_l2(o, o_ref) <= OUT_TOL and rel_l2(s, s_ref) <= STATE_TOL


# Heads whose state keeps a long memory (near-zero decay) or grows (g > 0) accumulate the bf16
# roundings of the W S product (W and the bf16 copy of S, ~2^-9 each) over that memory.  A CPU
# emulation of the kernel's roundings reproduces the GPU figures (1.46e-3 vs 1.68e-3 at decay 0.001,
# T=8192; 6.66e-3 vs 6.68e-3 for the growing head) and shows that the W S product sets them: S as
# bf16 hi + lo alone gives 1.22e-3, W and S in fp32 5.0e-4.  So these regimes are held to the
# bounds below, above the 1e-3 of the benchmark decays (whose state error is ~1e-4).
GROWING_STATE_TOL = 1.5e-3


def test_chunk_prefill_positive_g_heads(gdn, oracle, dev):
    """g > 0 (a growing state) on two of four value heads: the reference's decay e^{G_i - G_j} for
    i > j (src/gdn_chunk_fast2.py:41) has no sign condition.  2048 tokens (several segments: the
    growing heads take the exact summary path, the others warm up) and a one-chunk call.  Outputs
    within 1e-2; states within 1e-3 for the decaying heads and GROWING_STATE_TOL for the growing
    ones (head 1 grows ~e^8 over the 2048 tokens; measured 1.1e-3 there, 6.2e-4 on head 2: their
    chunks run W S in hi + lo, which took head 1 from 6.7e-3 to 1.9e-3, and the inverse's Gram
    matrix from the rounded normalised keys took it to 1.1e-3)."""
    for T, seed in ((2048, 31), (100, 32)):
        q, k, v, g, beta, s0 = _gdn_inputs(T, 2, 4, seed=seed)
        g[..., 1] = -g[..., 1] * 0.02        # (0, 0.01] per token: the state grows up to ~e^8
        g[..., 2] = -g[..., 2] * 0.005
        o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(_rep(q, 2), _rep(k, 2), v, g, beta, 64, s0, True, True)
        o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                                  initial_state=s0.to(dev), output_final_state=True,
                                                  use_qk_l2norm_in_kernel=True)
        for h in range(4):
            tol = GROWING_STATE_TOL if h in (1, 2) else STATE_TOL
            assert rel_l2(o[:, :, h], o_ref[:, :, h]) <= OUT_TOL, f"T {T} value head {h}"
            assert rel_l2(s[:, h], s_ref[:, h]) <= tol, (T, h, rel_l2(s[:, h], s_ref[:, h]))


@pytest.mark.parametrize("T", [8192, 32768])
def test_chunk_prefill_near_zero_decay_long(gdn, oracle, dev, T):
    """Near-zero decay (g ~ -0.002 per token: the state keeps ~500 tokens of memory) over long
    sequences, two value heads of one key head: outputs within 1e-2, final state within 1e-3
    (measured 4.9e-4 to 5.2e-4 at both lengths).  Every chunk here decays by less than e^-2 and runs
    W S in hi + lo; with the single bf16 product the state was 1.68e-3 off, and 8.1e-4 to 9.1e-4
    with the inverse's Gram matrix formed from the unrounded normalised keys."""
    q, k, v, g, beta, s0 = _gdn_inputs(T, 1, 2, seed=40 + T % 7, decay=0.001)
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(_rep(q, 2), _rep(k, 2), v, g, beta, 64, s0, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    for h in range(2):
        assert rel_l2(o[:, :, h], o_ref[:, :, h]) <= OUT_TOL, (h, rel_l2(o[:, :, h], o_ref[:, :, h]))
        assert rel_l2(s[:, h], s_ref[:, h]) <= STATE_TOL, (h, rel_l2(s[:, h], s_ref[:, h]))


def test_chunk_prefill_mixed_chunk_forms(gdn, oracle, dev):
    """Slow and fast decay alternating in runs of 96 tokens, so that chunks of one sequence switch
    between the hi + lo form of W S (decay over the chunk above e^-2) and the single bf16 product.
    Heads 0 and 2 (fast runs of g ~ -0.2) warm up; head 1 (fast runs of g ~ -0.05, about -7 over a
    4-chunk segment) leaves slots without a warm-up and takes the exact summary path; head 3 decays
    fast throughout.  Outputs within 1e-2, states within 1e-3."""
    T = 4096
    q, k, v, g, beta, s0 = _gdn_inputs(T, 2, 4, seed=55)
    slow = (torch.arange(T) // 96) % 2 == 0
    g[0, slow, :3] *= 0.01          # heads 0-2: g ~ -0.002 on the slow runs
    g[0, :, 1] *= 0.25
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(_rep(q, 2), _rep(k, 2), v, g, beta, 64, s0, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    for h in range(4):
        assert rel_l2(o[:, :, h], o_ref[:, :, h]) <= OUT_TOL, (h, rel_l2(o[:, :, h], o_ref[:, :, h]))
        assert rel_l2(s[:, h], s_ref[:, h]) <= STATE_TOL, (h, rel_l2(s[:, h], s_ref[:, h]))


def test_chunk_prefill_warm_up_and_exact_paths_per_head(gdn, oracle, dev):
    """Two packed sequences (2500 and 1596 tokens, 4-chunk segments at this size), value heads on each
    path the kernel can take for a later segment's initial state: strong decay (a one-chunk warm-up
    bounds the dropped state by 2^-16); moderate decay (a three-chunk warm-up); slow decay (no window
    within a segment reaches the bound: the exact summaries and combine, A formed); strong decay with
    one beta above 1 in the last chunk of a segment (the bound does not hold there: the exact path).
    Every head against the oracle."""
    lens = [2500, 1596]
    cu = torch.tensor([0, 2500, 4096], dtype=torch.int32)
    q, k, v, g, beta, _ = _gdn_inputs(4096, 2, 4, seed=21, state=False)
    g[..., 0] *= 10.0
    g[..., 1] *= 0.3
    g[..., 2] *= 0.05
    g[..., 3] *= 10.0
    beta[0, 1000, 3] = 1.5
    s0 = 0.02 * torch.randn(2, 4, 128, 128, generator=torch.Generator().manual_seed(22))
    o_ref, s_ref = oracle.chunk_gated_delta_rule_varlen(_rep(q, 2), _rep(k, 2), v, g, beta, cu, 64, s0, True, True)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev),
                                              initial_state=s0.to(dev), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(dev))
    for h in range(4):
        assert rel_l2(o[:, :, h], o_ref[:, :, h]) <= OUT_TOL, f"value head {h}"
        for i in range(len(lens)):
            assert rel_l2(s[i, h], s_ref[i, h]) <= STATE_TOL, f"sequence {i} value head {h}"


@pytest.mark.parametrize("lens", [[200, 1, 256, 130, 0, 64], [2500, 300, 1596]])
def test_chunk_prefill_seq_len_bound_matches_unknown(gdn, oracle, dev, lens):
    """Packed sequences through the C ABI with seq_len = 0 (no bound: the segment summaries are
    launched) and with seq_len = the longest sequence: bit-identical outputs and states, and against
    the oracle.  At 4 value heads these sizes cut segments of 4 chunks: in the first case no sequence
    spans two segments (the summaries are skipped), in the second two sequences do (kept)."""
    import importlib
    from conftest import PKG_NAME
    L = importlib.import_module(PKG_NAME + "._lib")
    Hk, Hv, D = 2, 4, 128
    T = sum(lens)
    q, k, v, g, beta, _ = _gdn_inputs(T, Hk, Hv, seed=31, state=False, decay=1.0)
    s0 = 0.02 * torch.randn(len(lens), Hv, D, D, generator=torch.Generator().manual_seed(32))
    cu_h = torch.tensor([0] + torch.cumsum(torch.tensor(lens), 0).tolist(), dtype=torch.int32)
    nch = [(n + 63) // 64 for n in lens]
    c0_h = torch.tensor([0] + torch.cumsum(torch.tensor(nch), 0).tolist(), dtype=torch.int32)
    total = int(c0_h[-1])
    qd, kd, vd, gd, bd = (x[0].contiguous().to(dev) for x in (q, k, v, g, beta))
    s0d, cu, c0 = s0.to(dev), cu_h.to(dev), c0_h.to(dev)
    work = torch.empty(int(L.lib().gdn_chunk_prefill_workspace_bytes(total, len(lens), Hv)), dtype=torch.uint8,
                       device=dev)
    res = []
    for bound in (0, max(lens)):
        out = torch.empty(T, Hv, D, dtype=torch.bfloat16, device=dev)
        fin = torch.empty_like(s0d)
        L.call("gdn_chunk_prefill", L.ptr(qd), qd.stride(0), L.ptr(kd), kd.stride(0), L.ptr(vd), vd.stride(0),
               L.ptr(gd), L.ptr(bd), L.BF16, L.ptr(s0d), L.ptr(fin), L.ptr(out), T, L.ptr(cu), L.ptr(c0), total,
               len(lens), bound, Hk, Hv, D, L.BF16, 1, L.ptr(work), work.numel(), L.stream_of(qd))
        torch.cuda.synchronize()
        res.append((out.clone(), fin.clone()))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    o_ref, s_ref = oracle.chunk_gated_delta_rule_varlen(_rep(q, 2), _rep(k, 2), v, g, beta, cu_h, 64, s0, True, True)
    assert rel_l2(res[1][0].cpu().unsqueeze(0), o_ref) <= OUT_TOL
    for i, n in enumerate(lens):
        if n:
            assert rel_l2(res[1][1][i].cpu(), s_ref[i]) <= STATE_TOL, f"sequence {i}"


@pytest.mark.parametrize("w_dtype,decay", [(torch.bfloat16, 0.1), (torch.float32, 0.1), (torch.bfloat16, 0.005)])
def test_chunk_prefill_fused_gated_norm_matches_two_calls(gdn, oracle, dev, w_dtype, decay):
    """The rule with its output rows passed through the gated RMSNorm in the output kernel against
    the rule followed by gdn_gated_rmsnorm: equal final states and bit-identical outputs (same sum
    order and roundings), and against the oracle.  Packed sequences of 1300, 5 and 900 tokens (at
    4 value heads, segments of 4 chunks; at decay 0.1 later segments start from a warm-up, at 0.005
    from the exact summaries and combine; a one-chunk sequence), gate rows from a wider tensor (row
    stride > Hv * d)."""
    import importlib
    from conftest import PKG_NAME
    engine = importlib.import_module(PKG_NAME + ".cb_engine")
    Hk, Hv, D = 2, 4, 128
    lens = [1300, 5, 900]
    T = sum(lens)
    cu = torch.tensor([0, 1300, 1305, 2205], dtype=torch.int32)
    q, k, v, g, beta, _ = _gdn_inputs(T, Hk, Hv, seed=41, state=False, decay=decay)
    s0 = 0.02 * torch.randn(3, Hv, D, D, generator=torch.Generator().manual_seed(42))
    g_ = torch.Generator().manual_seed(43)
    zw = torch.randn(T, Hv * D + 256, generator=g_).to(torch.bfloat16).to(dev)
    z = zw[:, 128:128 + Hv * D]
    nw = (1 + 0.1 * torch.randn(D, generator=g_)).to(w_dtype).to(dev)
    args = (q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev))
    kw = dict(initial_state=s0.to(dev), output_final_state=True, use_qk_l2norm_in_kernel=True,
              cu_seqlens=cu.to(dev))
    o, s = gdn.chunk_gated_delta_rule(*args, **kw)
    o2 = engine.gated_rmsnorm(o.reshape(T * Hv, D), z.reshape(T, Hv, D).reshape(T * Hv, D), nw, 1e-6)
    of, sf = gdn.chunk_gated_delta_rule(*args, **kw, norm_gate=(z, nw, 1e-6))
    assert torch.equal(s, sf)
    assert torch.equal(o2.reshape(T, Hv, D), of.reshape(T, Hv, D))
    o_ref, _ = oracle.chunk_gated_delta_rule_varlen(_rep(q, 2), _rep(k, 2), v, g, beta, cu, 64, s0, True, True)
    ref = oracle.gated_rmsnorm(o_ref.to(torch.bfloat16).reshape(T * Hv, D), z.cpu().reshape(T * Hv, D), nw.cpu())
    assert rel_l2(of.reshape(T * Hv, D), ref) <= OUT_TOL


@pytest.mark.parametrize("with_history", [False, True])
def test_conv_prefill(gdn, oracle, dev, with_history):
    C, K = 512, 4
    lens = [37, 2, 0, 130, 64]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    T = int(cu[-1])
    g_ = torch.Generator().manual_seed(17)
    x = torch.randn(T, C, generator=g_).to(torch.bfloat16)
    w = (0.5 * torch.randn(C, K, generator=g_)).to(torch.bfloat16)
    hist = torch.randn(len(lens), C, K, generator=g_).to(torch.bfloat16) if with_history else None
    out, st = gdn.causal_conv1d_prefill(x.t().unsqueeze(0).to(dev), w.to(dev), None,
                                        None if hist is None else hist.to(dev), cu.to(dev))
    out = out[0].t().cpu()
    for s in range(len(lens)):
        a, b = int(cu[s]), int(cu[s + 1])
        o_ref, st_ref = oracle.causal_conv1d_prefill(x[a:b].t().unsqueeze(0), w, None,
                                                     None if hist is None else hist[s:s + 1])
        assert torch.equal(st[s].cpu(), st_ref[0]), f"conv state of sequence {s}"
        if b > a:
            d = (out[a:b].float() - o_ref[0].t().float()).abs()
            assert (d <= o_ref[0].t().float().abs() * 2 ** -7 + 1e-6).all()


def test_prefill_core_then_decode_matches_oracle(gdn, oracle, dev):
    """Fused prefill layer (conv + gating + chunked rule + gated norm) on 3 packed prompts with conv
    history and initial state, then one fused decode step from the states it left."""
    Hk, Hv, D, K = 4, 8, 128, 4
    C = (2 * Hk + Hv) * D
    lens = [70, 128, 33]
    cu = torch.tensor([0, 70, 198, 231], dtype=torch.int32)
    T = 231
    g_ = torch.Generator().manual_seed(18)
    mixed = torch.randn(T, C, generator=g_).to(torch.bfloat16)
    z = torch.randn(T, Hv * D, generator=g_).to(torch.bfloat16)
    a = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    b = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    cw = (0.5 * torch.randn(C, K, generator=g_)).to(torch.bfloat16)
    A_log = torch.full((Hv,), -2.302585)
    dt = torch.full((Hv,), 2.0)
    nw = (1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16)
    hist = torch.randn(3, C, K, generator=g_).to(torch.bfloat16)
    s0 = 0.02 * torch.randn(3, Hv, D, D, generator=g_)
    core_ref, conv_ref, rec_ref = oracle.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D, cu,
                                                          hist, s0)
    dv = lambda x: x.to(dev)
    core, conv, rec = gdn.gdn_prefill_core(dv(mixed), dv(z), dv(a), dv(b), dv(cw), dv(A_log), dv(dt), dv(nw),
                                           Hk, Hv, D, cu_seqlens=dv(cu), conv_history=dv(hist),
                                           initial_state=dv(s0))
    assert torch.equal(conv.cpu(), conv_ref)
    assert rel_l2(core, core_ref) <= OUT_TOL and rel_l2(rec, rec_ref) <= STATE_TOL
    # one decode step for the 3 slots from the prefilled states
    m1 = torch.randn(3, C, generator=g_).to(torch.bfloat16)
    z1 = torch.randn(3, Hv * D, generator=g_).to(torch.bfloat16)
    a1 = torch.randn(3, Hv, generator=g_).to(torch.bfloat16)
    b1 = torch.randn(3, Hv, generator=g_).to(torch.bfloat16)
    cs_ref, rs_ref = conv_ref.clone(), rec_ref.clone()
    o_ref = oracle.gdn_decode_core(m1, z1, a1, b1, cs_ref, cw, A_log, dt, nw, rs_ref, Hk, Hv, D)
    o = gdn.gdn_decode_core(dv(m1), dv(z1), dv(a1), dv(b1), conv, dv(cw), dv(A_log), dv(dt), dv(nw), rec,
                            Hk, Hv, D)
    assert torch.equal(conv.cpu(), cs_ref)
    assert rel_l2(o, o_ref) <= OUT_TOL and rel_l2(rec, rs_ref) <= STATE_TOL


def test_prefill_core_long_memory_heads(gdn, oracle, dev):
    """The fused prefill layer with decays from near zero to fast across heads: exp(A_log) from 0.001
    to 3 with dt_bias 0, so g runs from ~ -0.0007 to ~ -2 a token.  Heads 0-3 decay by less than e^-2
    over a chunk (W S in hi + lo) and leave the 1500-token prompt's segment boundaries without a
    warm-up (exact summary path, summaries without the norm, outputs with it); heads 4-7 warm up.
    Against the oracle's composition: outputs within 1e-2, states within 1e-3, conv states exact."""
    Hk, Hv, D, K = 4, 8, 128, 4
    C = (2 * Hk + Hv) * D
    cu = torch.tensor([0, 1500, 2400, 2464, 3164], dtype=torch.int32)
    T = 3164
    g_ = torch.Generator().manual_seed(71)
    mixed = torch.randn(T, C, generator=g_).to(torch.bfloat16)
    z = torch.randn(T, Hv * D, generator=g_).to(torch.bfloat16)
    a = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    b = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    cw = (0.5 * torch.randn(C, K, generator=g_)).to(torch.bfloat16)
    A_log = torch.log(torch.tensor([0.001, 0.003, 0.01, 0.03, 0.1, 0.3, 1.0, 3.0]))
    dt = torch.zeros(Hv)
    nw = (1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16)
    hist = torch.randn(4, C, K, generator=g_).to(torch.bfloat16)
    s0 = 0.02 * torch.randn(4, Hv, D, D, generator=g_)
    core_ref, conv_ref, rec_ref = oracle.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D, cu,
                                                          hist, s0)
    dv = lambda x: x.to(dev)
    core, conv, rec = gdn.gdn_prefill_core(dv(mixed), dv(z), dv(a), dv(b), dv(cw), dv(A_log), dv(dt), dv(nw),
                                           Hk, Hv, D, cu_seqlens=dv(cu), conv_history=dv(hist),
                                           initial_state=dv(s0))
    torch.cuda.synchronize()
    assert torch.equal(conv.cpu(), conv_ref)
    co, co_ref = core.reshape(T, Hv, D), core_ref.reshape(T, Hv, D)
    for h in range(Hv):
        assert rel_l2(co[:, h], co_ref[:, h]) <= OUT_TOL, (h, rel_l2(co[:, h], co_ref[:, h]))
        assert rel_l2(rec[:, h], rec_ref[:, h]) <= STATE_TOL, (h, rel_l2(rec[:, h], rec_ref[:, h]))


def test_conv_silu_every_bf16_input(gdn, oracle, dev):
    """The conv's SiLU rounds to bf16 as torch does (fp32 x / (1 + e^-x), one rounding), bit for bit,
    for every normal bf16 input: one token through the taps (0, 0, 0, 1), so the conv's bf16 output
    before the SiLU is the input itself.  A one-ulp slip on a few inputs (x = -2^-8 and 2^-7 among
    them) moves a fast-decaying head's final state by up to 7e-3 when it hits a sequence's last token.
    The fused layer's prologue runs the same conv code."""
    x = normal_bf16_values()
    x = torch.cat([x, torch.zeros(-x.numel() % 8, dtype=x.dtype)])  # whole 8-channel groups
    C, K = x.numel(), 4
    w = torch.zeros(C, K, dtype=torch.bfloat16)
    w[:, K - 1] = 1
    out, _ = gdn.causal_conv1d_prefill(x.reshape(1, C, 1).to(dev), w.to(dev))
    ref, _ = oracle.causal_conv1d_prefill(x.reshape(1, C, 1), w)
    assert_same_bits(out, ref, x)


def test_gating_every_bf16_input(gdn, oracle, dev):
    """beta = sigmoid(b) rounds to bf16 as torch does, bit for bit, for every normal bf16 b (b = -2^-8
    and 2^-7 lie within an fp32 ulp of a bf16 rounding midpoint)."""
    b = normal_bf16_values()
    b = b[:b.numel() - b.numel() % 15].reshape(-1, 15)
    a = torch.zeros_like(b)
    zeros = torch.zeros(15)
    beta_ref, _ = oracle.gdn_gating(a, b, zeros, zeros)
    beta, _ = gdn.gdn_gating(a.to(dev), b.to(dev), zeros.to(dev), zeros.to(dev))
    assert_same_bits(beta, beta_ref, b)


def test_gating(gdn, oracle, dev):
    g_ = torch.Generator().manual_seed(19)
    a = torch.randn(50, 32, generator=g_).to(torch.bfloat16)
    b = torch.randn(50, 32, generator=g_).to(torch.bfloat16)
    A_log = torch.log(torch.rand(32, generator=g_) * 16 + 0.1)
    dt = torch.rand(32, generator=g_)
    beta_ref, g_ref = oracle.gdn_gating(a, b, A_log, dt)
    beta, g = gdn.gdn_gating(a.to(dev), b.to(dev), A_log.to(dev), dt.to(dev))
    assert torch.equal(beta.cpu(), beta_ref)
    assert rel_l2(g, g_ref) <= 1e-6

