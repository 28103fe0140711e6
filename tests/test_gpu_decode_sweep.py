"""A seeded sweep of the fused decode layer (gdn_decode_core: conv update + SiLU, gating, l2norm,
recurrent step, gated RMSNorm in one kernel) over 1-8 consecutive decode steps, against the oracle's
composition of the same steps (src/cb_engine.py:318-352 with ELEM_CONV): slot counts 1-32 (odd ones
included), key heads 1-16 read by 1-4 value heads each, conv kernels of 2-4 taps, inputs and conv
windows at scale 0.3, 1 or 3, conv bias every third case, decay rates exp(A_log) down to 1e-4 with
dt_bias up to 3 N(0, 1), states of scale 0.02 or 0.5, bf16 and fp32 norm weights.  After every step the
conv state is the oracle's bit for bit and each slot's output is within 1e-2 rel-L2; after the last
step every (slot, value head) state is within 1e-3.  Measured worst over these cases: outputs 1.1e-3,
states 5.6e-7.
"""
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu

D = 128


def _case(i):
    r = torch.Generator().manual_seed(300000 + i)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=r))]
    N = pick([1, 2, 3, 7, 16, 17, 32])
    Hk = pick([1, 2, 4, 8, 16])
    Hv = Hk * pick([1, 2, 3, 4])
    return N, Hk, Hv, pick([2, 3, 4, 4]), pick([0.3, 1.0, 3.0]), pick([1, 3, 8]), r


@pytest.mark.parametrize("i", range(30))
def test_decode_layer_sweep(gdn, oracle, dev, i):
    N, Hk, Hv, K, xs, steps, r = _case(i)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=r))]
    C, bf = (2 * Hk + Hv) * D, torch.bfloat16
    g_ = torch.Generator().manual_seed(350000 + i)
    cw = (0.5 * torch.randn(C, K, generator=g_)).to(bf)
    A_log = torch.log(torch.rand(Hv, generator=g_) * pick([0.01, 1.0, 5.0]) + 1e-4)
    dt = pick([0.0, 1.0, 3.0]) * torch.randn(Hv, generator=g_)
    nw = (1 + 0.1 * torch.randn(D, generator=g_)).to(bf if i % 2 else torch.float32)
    bias = (0.5 * torch.randn(C, generator=g_)).to(bf) if i % 3 == 0 else None
    ref_conv = (xs * torch.randn(N, C, K, generator=g_)).to(bf)
    ref_rec = pick([0.02, 0.5]) * torch.randn(N, Hv, D, D, generator=g_)
    conv, rec = ref_conv.to(dev), ref_rec.to(dev)
    print(f"decode case {i}: N {N} Hk {Hk} Hv {Hv} K {K} scale {xs} steps {steps} bias {bias is not None}", flush=True)
    on = lambda x: None if x is None else x.to(dev)
    for st in range(steps):
        mixed = (xs * torch.randn(N, C, generator=g_)).to(bf)
        z = (2 * torch.randn(N, Hv * D, generator=g_)).to(bf)
        a = (2 * torch.randn(N, Hv, generator=g_)).to(bf)
        b = (2 * torch.randn(N, Hv, generator=g_)).to(bf)
        ref = oracle.gdn_decode_core(mixed, z, a, b, ref_conv, cw, A_log, dt, nw, ref_rec, Hk, Hv, D, conv_bias=bias)
        out = gdn.gdn_decode_core(on(mixed), on(z), on(a), on(b), conv, on(cw), on(A_log), on(dt), on(nw), rec, Hk, Hv,
                                  D, conv_bias=on(bias))
        torch.cuda.synchronize()
        assert torch.equal(conv.cpu(), ref_conv), f"conv state, step {st}"
        for n in range(N):
            assert rel_l2(out[n], ref[n]) <= 1e-2, (st, n, rel_l2(out[n], ref[n]))
    for n in range(N):
        for h in range(Hv):
            assert rel_l2(rec[n, h], ref_rec[n, h]) <= 1e-3, (n, h, rel_l2(rec[n, h], ref_rec[n, h]))
