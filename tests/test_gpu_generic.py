"""GPU parity of the generic chunked prefill (gdn_chunk_prefill_generic: any head dims in
{16, 32, 64, 128}, fp32 / bf16 / fp16 inputs, fp32 arithmetic) -- the reference's
fast_chunk_gated_delta_rule_v2 is generic in dtype and head dims (src/gdn_chunk_fast2.py:11-29).

The reference's CPU-runnable case (B=1, T=512, H=4, d=64, fp32, chunk 64, seed 0) is run exactly,
against the oracle's token-by-token recurrence and its chunked v2.  With fp32 inputs everything is
fp32, so the bar is tighter than the bf16 one: output and final state within 1e-4 rel-L2 (the two
fp32 CPU paths themselves differ by about 1e-6).  Inputs in bf16 / fp16 keep the bf16 bar:
output <= 1e-2, state <= 1e-3 rel-L2.
"""
import pytest
import torch
import torch.nn.functional as F

from conftest import rel_l2

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4


def config0(seed=0, T=512, H=4, d=64):
    """B=1, T=512, H=4, d=64, fp32; q,k ~N(0,1) l2-normalised per head, v ~N(0,1),
    beta = sigmoid(N(0,1)), g = -softplus(N(0,1)+2)*0.1, zero initial state, seed 0."""
    g_ = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(1, T, H, d, generator=g_), dim=-1)
    k = F.normalize(torch.randn(1, T, H, d, generator=g_), dim=-1)
    v = torch.randn(1, T, H, d, generator=g_)
    beta = torch.sigmoid(torch.randn(1, T, H, generator=g_))
    g = -F.softplus(torch.randn(1, T, H, generator=g_) + 2) * 0.1
    return q, k, v, g, beta


def _dev(dev, *xs):
    return [None if x is None else x.to(dev) for x in xs]


def test_config0_exactly(gdn, oracle, dev):
    """Config 0 on the HIP path: chunked (the drop-in v2 name) against the oracle's token recurrence
    (the closed-form equivalence that pins the chunked rule) and its chunked v2, zero initial state."""
    q, k, v, g, beta = config0()
    o_rec, s_rec = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, None, True, False)
    o_chk, s_chk = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, None, True, False)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(*_dev(dev, q, k, v, g, beta), chunk_size=64, initial_state=None,
                                              output_final_state=True, use_qk_l2norm_in_kernel=False)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and o.shape == (1, 512, 4, 64) and s.shape == (1, 4, 64, 64)
    for ref_o, ref_s in ((o_rec, s_rec), (o_chk, s_chk)):
        assert rel_l2(o, ref_o) <= FP32_TOL, rel_l2(o, ref_o)
        assert rel_l2(s, ref_s) <= FP32_TOL, rel_l2(s, ref_s)
    # the v1 name and in-kernel l2norm on the raw draws give the same rule
    g_ = torch.Generator().manual_seed(0)
    qr = torch.randn(1, 512, 4, 64, generator=g_)
    kr = torch.randn(1, 512, 4, 64, generator=g_)
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v1(qr, kr, v, g, beta, 64, None, True, True)
    o1, s1 = gdn.fast_chunk_gated_delta_rule(*_dev(dev, qr, kr, v, g, beta), output_final_state=True,
                                             use_qk_l2norm_in_kernel=True)
    assert rel_l2(o1, o_ref) <= FP32_TOL and rel_l2(s1, s_ref) <= FP32_TOL


@pytest.mark.parametrize("chunk_size", [16, 32, 128])
def test_any_chunk_size_gives_the_same_rule(gdn, oracle, dev, chunk_size):
    """The reference honours chunk_size (src/gdn_chunk_fast2.py:22-37); every chunk size is the same
    recurrence, and the kernels compute it with 64-token chunks."""
    q, k, v, g, beta = config0(seed=3, T=300)
    s0 = 0.02 * torch.randn(1, 4, 64, 64, generator=torch.Generator().manual_seed(4))
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, chunk_size, s0, True, False)
    o, s = gdn.fast_chunk_gated_delta_rule_v2(*_dev(dev, q, k, v, g, beta), chunk_size=chunk_size,
                                              initial_state=s0.to(dev), output_final_state=True)
    assert rel_l2(o, o_ref) <= FP32_TOL and rel_l2(s, s_ref) <= FP32_TOL


@pytest.mark.parametrize("dtype,Dk,Dv,T,Hk,Hv", [
    (torch.float32, 128, 128, 200, 2, 4),     # fp32 at the model's head dim: two value slices
    (torch.float32, 32, 16, 130, 1, 3),       # d_k != d_v, a value slice of 16 columns
    (torch.bfloat16, 64, 64, 257, 2, 2),      # bf16 at d = 64
    (torch.float16, 32, 64, 65, 2, 4),        # fp16
    (torch.bfloat16, 128, 64, 150, 1, 2),     # bf16 with d_v != 128: not the fast path
    (torch.float32, 16, 16, 1, 1, 1),         # one token
])
def test_generic_dtypes_and_head_dims(gdn, oracle, dev, dtype, Dk, Dv, T, Hk, Hv):
    g_ = torch.Generator().manual_seed(T * 7 + Dk + Dv)
    q = torch.randn(1, T, Hk, Dk, generator=g_).to(dtype)
    k = torch.randn(1, T, Hk, Dk, generator=g_).to(dtype)
    v = torch.randn(1, T, Hv, Dv, generator=g_).to(dtype)
    beta = torch.sigmoid(torch.randn(1, T, Hv, generator=g_)).to(dtype)
    g = -F.softplus(torch.randn(1, T, Hv, generator=g_) + 2) * 0.1
    s0 = 0.02 * torch.randn(1, Hv, Dk, Dv, generator=g_)
    r = Hv // Hk
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q.repeat_interleave(r, 2), k.repeat_interleave(r, 2), v, g, beta,
                                                    64, s0, True, True)
    o, s = gdn.chunk_gated_delta_rule(*_dev(dev, q, k, v, g, beta), initial_state=s0.to(dev),
                                      output_final_state=True, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert o.dtype == dtype and o.shape == (1, T, Hv, Dv)
    otol, stol = (FP32_TOL, FP32_TOL) if dtype == torch.float32 else (1e-2, 1e-3)
    assert rel_l2(o, o_ref) <= otol, rel_l2(o, o_ref)
    assert rel_l2(s, s_ref) <= stol, rel_l2(s, s_ref)


def test_generic_varlen_and_slot_rows(gdn, oracle, dev):
    """Packed sequences (one empty, one of 1 token) through cu_seqlens, states in slot rows (initial and
    final the same buffer, an untouched spare row), fp32 at d = 64: each sequence equals its own call."""
    lens, Hk, Hv, D = [100, 0, 1, 190], 2, 4, 64
    T = sum(lens)
    g_ = torch.Generator().manual_seed(21)
    q = torch.randn(1, T, Hk, D, generator=g_)
    k = torch.randn(1, T, Hk, D, generator=g_)
    v = torch.randn(1, T, Hv, D, generator=g_)
    beta = torch.sigmoid(torch.randn(1, T, Hv, generator=g_))
    g = -F.softplus(torch.randn(1, T, Hv, generator=g_) + 2) * 0.1
    slots = torch.randn(6, Hv, D, D, generator=g_) * 0.02
    rows = [4, 0, 2, 5]
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    sd = slots.to(dev)
    o, _ = gdn.chunk_gated_delta_rule(*_dev(dev, q, k, v, g, beta), initial_state=sd, cu_seqlens=cu,
                                      state_rows=rows, final_state_out=sd, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    r = Hv // Hk
    for i, L in enumerate(lens):
        a, b = cu[i], cu[i + 1]
        sl = slice(a, b)
        o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q[:, sl].repeat_interleave(r, 2), k[:, sl].repeat_interleave(r, 2),
                                                        v[:, sl], g[:, sl], beta[:, sl], 64, slots[rows[i]][None],
                                                        True, True)
        if L:
            assert rel_l2(o[:, sl], o_ref) <= FP32_TOL
        assert rel_l2(sd[rows[i]], s_ref[0]) <= FP32_TOL
    for spare in (1, 3):
        assert torch.equal(sd[spare].cpu(), slots[spare]), "a row no sequence names must stay untouched"


def test_generic_refusals(gdn, dev):
    """Outside the reference's domain: mixed dtypes, float64, head dims outside {16, 32, 64, 128}, the fused
    norm on the generic path, a bad chunk size -- ValueError before any launch."""
    x = torch.zeros(1, 4, 2, 64, device=dev)
    gg = torch.zeros(1, 4, 2, device=dev)
    with pytest.raises(ValueError, match="dtypes"):
        gdn.chunk_gated_delta_rule(x, x, x.to(torch.bfloat16), gg, gg)
    with pytest.raises(ValueError, match="dtypes"):
        gdn.chunk_gated_delta_rule(x.double(), x.double(), x.double(), gg, gg)
    x96 = torch.zeros(1, 4, 2, 96, device=dev)
    with pytest.raises(ValueError, match="head dims"):
        gdn.chunk_gated_delta_rule(x96, x96, x96, gg, gg)
    with pytest.raises(ValueError, match="chunk_size"):
        gdn.chunk_gated_delta_rule(x, x, x, gg, gg, chunk_size=0)
    with pytest.raises(ValueError, match="fused output norm"):
        gdn.chunk_gated_delta_rule(x, x, x, gg, gg, norm_gate=(torch.zeros(4, 128, device=dev), None, 1e-6))


@pytest.mark.parametrize("i", range(40))
def test_generic_sweep(gdn, oracle, dev, i):
    """A seeded sweep over the drop-in's generic signature: fp32 / bf16 / fp16 inputs, head dims
    d_k, d_v in {16, 32, 64, 128}, 1-4 key heads read by 1-3 value heads, batches of 1-3 sequences of
    1-700 tokens, l2norm in or out of the kernel, decay scales 0.001-1, chunk sizes 16-128, zero or
    random initial states.  fp32 within 1e-4 rel-L2 (output and state); bf16 / fp16 within 1e-2 /
    1e-3.  Measured worst: fp32 1.4e-6 / 3.8e-6, fp16 1.7e-5 / 7.8e-6, bf16 3.3e-3 / 4.5e-6."""
    r = torch.Generator().manual_seed(400000 + i)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=r))]
    dtype = pick([torch.float32, torch.bfloat16, torch.float16])
    Dk, Dv = pick([16, 32, 64, 128]), pick([16, 32, 64, 128])
    Hk = pick([1, 2, 4])
    Hv = Hk * pick([1, 2, 3])
    B, T = pick([1, 2, 3]), pick([1, 2, 63, 64, 65, 130, 300, 700])
    l2, decay, chunk = pick([True, False]), pick([0.001, 0.1, 1.0]), pick([16, 32, 64, 128])
    g_ = torch.Generator().manual_seed(470000 + i)
    q, k = torch.randn(B, T, Hk, Dk, generator=g_), torch.randn(B, T, Hk, Dk, generator=g_)
    if not l2:
        q, k = F.normalize(q, dim=-1), F.normalize(k, dim=-1)
    q, k = q.to(dtype), k.to(dtype)
    v = torch.randn(B, T, Hv, Dv, generator=g_).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=g_)).to(dtype)
    g = -F.softplus(torch.randn(B, T, Hv, generator=g_) + 2) * decay
    s0 = 0.02 * torch.randn(B, Hv, Dk, Dv, generator=g_) if i % 2 else None
    print(f"generic case {i}: {dtype} Dk {Dk} Dv {Dv} Hk {Hk} Hv {Hv} B {B} T {T} l2 {l2} decay {decay} "
          f"chunk {chunk}", flush=True)
    r_ = Hv // Hk
    o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(q.repeat_interleave(r_, 2), k.repeat_interleave(r_, 2), v, g, beta,
                                                    chunk, s0, True, l2)
    o, s = gdn.chunk_gated_delta_rule(*_dev(dev, q, k, v, g, beta), chunk_size=chunk,
                                      initial_state=None if s0 is None else s0.to(dev), output_final_state=True,
                                      use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    assert o.dtype == dtype and o.shape == (B, T, Hv, Dv)
    otol, stol = (FP32_TOL, FP32_TOL) if dtype == torch.float32 else (1e-2, 1e-3)
    assert rel_l2(o.float(), o_ref.float()) <= otol, rel_l2(o.float(), o_ref.float())
    assert rel_l2(s, s_ref) <= stol, rel_l2(s, s_ref)
