"""GPU tests of the continuous-batching slot paths: prefill whose conv and recurrent states go
straight into slot rows (fresh and continuation chunks, src/cb_engine.py:198-205,
src/cb_tp.py:153-263), and the masked decode step that leaves held slots untouched
(src/cb_tp.py:274-285).  Each path is checked against the oracle's compositions on the same inputs
(outputs rel-L2 <= 1e-2, fp32 states <= 1e-3, conv states bit for bit), and against the plain HIP
call for the properties of the slot layout itself (rows written bit-identical to the plain call's
states, other rows untouched)."""
import pytest
import torch

from conftest import rel_l2

OUT_TOL, STATE_TOL = 1e-2, 1e-3
Hk, Hv, D, K = 4, 8, 128, 4
C = (2 * Hk + Hv) * D


def _layer_inputs(T, seed):
    g_ = torch.Generator().manual_seed(seed)
    mixed = torch.randn(T, C, generator=g_).to(torch.bfloat16)
    z = torch.randn(T, Hv * D, generator=g_).to(torch.bfloat16)
    a = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    b = torch.randn(T, Hv, generator=g_).to(torch.bfloat16)
    return mixed, z, a, b


def _params(seed):
    g_ = torch.Generator().manual_seed(seed)
    cw = (0.5 * torch.randn(C, K, generator=g_)).to(torch.bfloat16)
    A_log = torch.full((Hv,), -2.302585)
    dt = torch.full((Hv,), 2.0)
    nw = (1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16)
    return cw, A_log, dt, nw


def _cpu(*ts):
    return [t.cpu() for t in ts]


@pytest.mark.gpu
def test_prefill_into_slot_rows(gdn, oracle, dev):
    """3 packed prompts into slots [5, 0, 3] of an 8-slot engine: those rows equal the plain call's
    states bit for bit, every other row is untouched."""
    cu = torch.tensor([0, 70, 198, 231], dtype=torch.int32)
    T = 231
    mixed, z, a, b = (x.to(dev) for x in _layer_inputs(T, 30))
    cw, A_log, dt, nw = (x.to(dev) for x in _params(31))
    cud = cu.to(dev)
    core_ref, conv_ref, rec_ref = gdn.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D,
                                                       cu_seqlens=cud)
    g_ = torch.Generator().manual_seed(32)
    conv_slots = torch.randn(8, C, K, generator=g_).to(torch.bfloat16).to(dev)
    rec_slots = torch.randn(8, Hv, D, D, generator=g_).to(dev)
    conv0, rec0 = conv_slots.clone(), rec_slots.clone()
    # host lengths and rows (no GPU wait) must give what device ones give
    core, cs, rs = gdn.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D, cu_seqlens=cu,
                                        slots=[5, 0, 3], conv_slots=conv_slots, rec_slots=rec_slots)
    assert cs is conv_slots and rs is rec_slots
    assert torch.equal(core, core_ref)
    for i, r in enumerate([5, 0, 3]):
        assert torch.equal(conv_slots[r], conv_ref[i]) and torch.equal(rec_slots[r], rec_ref[i])
    for r in (1, 2, 4, 6, 7):
        assert torch.equal(conv_slots[r], conv0[r]) and torch.equal(rec_slots[r], rec0[r])
    # the oracle's composition (src/cb_tp.py:153-181 per prompt) on the same inputs
    o_core, o_conv, o_rec = oracle.gdn_prefill_core(*_cpu(mixed, z, a, b, cw, A_log, dt, nw), Hk, Hv, D,
                                                    cu_seqlens=cu)
    assert rel_l2(core, o_core) <= OUT_TOL
    for i, r in enumerate([5, 0, 3]):
        assert torch.equal(conv_slots[r].cpu(), o_conv[i]) and rel_l2(rec_slots[r], o_rec[i]) <= STATE_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("split", [1, 2, 64, 100])
def test_prefill_continuation_through_slots(gdn, oracle, dev, split):
    """A prompt prefilled in two chunks through its slot row (the second chunk reads the conv history
    and recurrent state the first left there, src/cb_tp.py:230-263) matches one pass."""
    T = 150
    mixed, z, a, b = (x.to(dev) for x in _layer_inputs(T, 33))
    cw, A_log, dt, nw = (x.to(dev) for x in _params(34))
    core_ref, conv_ref, rec_ref = gdn.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D)
    conv_slots = torch.zeros(4, C, K, dtype=torch.bfloat16, device=dev)
    rec_slots = torch.zeros(4, Hv, D, D, device=dev)
    slots = torch.tensor([2], dtype=torch.int32, device=dev)
    parts = []
    for lo, hi, cont in ((0, split, False), (split, T, True)):
        c, _, _ = gdn.gdn_prefill_core(mixed[lo:hi], z[lo:hi], a[lo:hi], b[lo:hi], cw, A_log, dt, nw, Hk, Hv, D,
                                       slots=slots, conv_slots=conv_slots, rec_slots=rec_slots,
                                       continuation=cont)
        parts.append(c)
    core = torch.cat(parts)
    assert torch.equal(conv_slots[2], conv_ref[0])  # the conv window is pure data movement
    assert rel_l2(core, core_ref) <= OUT_TOL and rel_l2(rec_slots[2], rec_ref[0]) <= STATE_TOL
    assert torch.count_nonzero(conv_slots[[0, 1, 3]]) == 0 and torch.count_nonzero(rec_slots[[0, 1, 3]]) == 0
    # the oracle's continuation (src/cb_tp.py:230-263): the second chunk starts from the first's conv
    # window and recurrent state
    xs = _cpu(mixed, z, a, b)
    ps = _cpu(cw, A_log, dt, nw)
    c1, cs1, rs1 = oracle.gdn_prefill_core(*(x[:split] for x in xs), *ps, Hk, Hv, D)
    c2, cs2, rs2 = oracle.gdn_prefill_core(*(x[split:] for x in xs), *ps, Hk, Hv, D, conv_history=cs1,
                                           initial_state=rs1)
    assert rel_l2(parts[0], c1) <= OUT_TOL and rel_l2(parts[1], c2) <= OUT_TOL
    assert torch.equal(conv_slots[2].cpu(), cs2[0]) and rel_l2(rec_slots[2], rs2[0]) <= STATE_TOL


@pytest.mark.gpu
def test_decode_masked_slots(gdn, oracle, dev):
    """A dense decode step with held slots: held rows keep their conv and recurrent state bit for bit
    and output zeros; active rows equal the unmasked step's."""
    N = 5
    mixed, z, a, b = (x.to(dev) for x in _layer_inputs(N, 35))
    cw, A_log, dt, nw = (x.to(dev) for x in _params(36))
    g_ = torch.Generator().manual_seed(37)
    conv0 = torch.randn(N, C, K, generator=g_).to(torch.bfloat16).to(dev)
    rec0 = (0.02 * torch.randn(N, Hv, D, D, generator=g_)).to(dev)
    cs_ref, rs_ref = conv0.clone(), rec0.clone()
    o_ref = gdn.gdn_decode_core(mixed, z, a, b, cs_ref, cw, A_log, dt, nw, rs_ref, Hk, Hv, D)
    active = torch.tensor([1, 0, 1, 1, 0], dtype=torch.bool, device=dev)
    cs, rs = conv0.clone(), rec0.clone()
    o = gdn.gdn_decode_core(mixed, z, a, b, cs, cw, A_log, dt, nw, rs, Hk, Hv, D, active=active)
    for n in range(N):
        if active[n]:
            assert torch.equal(o[n], o_ref[n]) and torch.equal(cs[n], cs_ref[n]) and torch.equal(rs[n], rs_ref[n])
        else:
            assert torch.count_nonzero(o[n]) == 0
            assert torch.equal(cs[n], conv0[n]) and torch.equal(rs[n], rec0[n])
    # the active rows against the oracle's decode layer on those rows alone
    act = [n for n in range(N) if active[n]]
    c_o, r_o = conv0[act].cpu(), rec0[act].cpu()
    o_o = oracle.gdn_decode_core(*(x[act].cpu() for x in (mixed, z, a, b)), c_o, *_cpu(cw, A_log, dt, nw), r_o,
                                 Hk, Hv, D)
    assert rel_l2(o[act], o_o) <= OUT_TOL
    assert torch.equal(cs[act].cpu(), c_o) and rel_l2(rs[act], r_o) <= STATE_TOL


def _composed_layer(gdn, mixed, z, a, b, cw, A_log, dt, nw, cu, hist=None, init=None, rows=None, conv_slots=None,
                    rec_slots=None, cont=False, bias=None):
    """The prefill layer as separate calls: conv prefill, gating, the chunked rule with the fused norm."""
    T = mixed.shape[0]
    if rows is not None:
        conv_out, conv_state = gdn.causal_conv1d_prefill(mixed.t().unsqueeze(0), cw, bias,
                                                         conv_slots if cont else None, cu, state_rows=rows,
                                                         state_out=conv_slots)
    else:
        conv_out, conv_state = gdn.causal_conv1d_prefill(mixed.t().unsqueeze(0), cw, bias, hist, cu)
    qkv = conv_out[0].t()
    kd = Hk * D
    q, k, v = (qkv[:, :kd].reshape(1, T, Hk, D), qkv[:, kd:2 * kd].reshape(1, T, Hk, D),
               qkv[:, 2 * kd:].reshape(1, T, Hv, D))
    beta, g = gdn.gdn_gating(a.reshape(1, T, Hv), b.reshape(1, T, Hv), A_log, dt)
    if rows is not None:
        core, rec = gdn.chunk_gated_delta_rule(q, k, v, g, beta, 64, rec_slots if cont else None, True, True,
                                               cu_seqlens=cu, state_rows=rows, final_state_out=rec_slots,
                                               norm_gate=(z, nw, 1e-6))
    else:
        core, rec = gdn.chunk_gated_delta_rule(q, k, v, g, beta, 64, init, True, True, cu_seqlens=cu,
                                               norm_gate=(z, nw, 1e-6))
    return core.reshape(T, Hv * D), conv_state, rec


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fresh", "history", "history_f32_norm_bias", "slots_continued"])
def test_prefill_layer_entry_matches_separate_calls(gdn, dev, mode):
    """gdn_prefill_core (one gdn_prefill_layer_rows call: conv, conv state, gating and segment table
    in one launch) against the same layer as separate calls, bit for bit: outputs, conv states and
    recurrent states.  Packed prompts of 300, 1, 0 and 777 tokens; fresh (zero history), with an
    explicit conv history and initial states (also with an fp32 norm weight and a conv bias), and
    through slot rows continuing a previous chunk (history rows = state rows: the conv state is
    captured by a launch of its own)."""
    lens = [300, 1, 0, 777]
    cu = torch.tensor([0, 300, 301, 301, 1078], dtype=torch.int32)
    T = 1078
    mixed, z, a, b = (t.to(dev) for t in _layer_inputs(T, 61))
    cw, A_log, dt, nw = (t.to(dev) for t in _params(62))
    g_ = torch.Generator().manual_seed(63)
    bias = None
    if mode == "history_f32_norm_bias":
        nw = nw.float() + 0.01
        bias = (0.1 * torch.randn(C, generator=g_)).to(torch.bfloat16).to(dev)
    if mode == "slots_continued":
        N = 6
        slots = torch.tensor([4, 0, 2, 5], dtype=torch.int32)
        cs0 = torch.randn(N, C, K, generator=g_).to(torch.bfloat16).to(dev)
        rs0 = (0.02 * torch.randn(N, Hv, D, D, generator=g_)).to(dev)
        cs1, rs1 = cs0.clone(), rs0.clone()
        o1, c1, r1 = gdn.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D, cu_seqlens=cu, slots=slots,
                                          conv_slots=cs1, rec_slots=rs1, continuation=True)
        cs2, rs2 = cs0.clone(), rs0.clone()
        o2, c2, r2 = _composed_layer(gdn, mixed, z, a, b, cw, A_log, dt, nw, cu.to(dev), rows=slots,
                                     conv_slots=cs2, rec_slots=rs2, cont=True)
    else:
        hist = init = None
        if mode != "fresh":
            hist = torch.randn(len(lens), C, K, generator=g_).to(torch.bfloat16).to(dev)
            init = (0.02 * torch.randn(len(lens), Hv, D, D, generator=g_)).to(dev)
        o1, c1, r1 = gdn.gdn_prefill_core(mixed, z, a, b, cw, A_log, dt, nw, Hk, Hv, D, cu_seqlens=cu,
                                          conv_history=hist, initial_state=init, conv_bias=bias)
        o2, c2, r2 = _composed_layer(gdn, mixed, z, a, b, cw, A_log, dt, nw, cu.to(dev), hist=hist, init=init,
                                     bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(c1, c2)
    assert torch.equal(r1, r2)
