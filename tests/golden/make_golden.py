"""Writes the golden fixtures in this folder from the CPU oracle (run: python tests/golden/make_golden.py).

Every prefill vector is cross-checked against transformers' torch_chunk_gated_delta_rule and the
decode vector against torch_recurrent_gated_delta_rule before it is written.  bf16 tensors are
stored as their uint16 bit patterns.  Shapes are the smallest that exercise the kernels' real head
dim (d = 128): T in {1, 63, 64, 65, 130} covers empty, partial, exact and multi-chunk prefill.
"""
import importlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
O = importlib.import_module("oracle.gdn_oracle")
HF = importlib.import_module("transformers.models.qwen3_5.modeling_qwen3_5")


def bits(t):
    return t.contiguous().view(torch.int16).numpy().astype(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def prefill(T, with_state, seed):
    g_ = torch.Generator().manual_seed(seed)
    D = 128
    q = torch.randn(1, T, 1, D, generator=g_).to(torch.bfloat16)
    k = torch.randn(1, T, 1, D, generator=g_).to(torch.bfloat16)
    v = torch.randn(1, T, 1, D, generator=g_).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(1, T, 1, generator=g_)).to(torch.bfloat16)
    g = -torch.nn.functional.softplus(torch.randn(1, T, 1, generator=g_) + 2) * 0.1
    s0 = 0.02 * torch.randn(1, 1, D, D, generator=g_) if with_state else torch.zeros(1, 1, D, D)
    o, s = O.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, s0, True, True)
    # transformers' chunk rule on the oracle's l2-normalised q, k (its own bf16 l2norm rounds some
    # rows one ulp differently depending on their position in torch's vectorised loop)
    o_hf, s_hf = HF.torch_chunk_gated_delta_rule(O.l2norm(q), O.l2norm(k), v, g, beta, 64, s0, True, False)
    assert rel(o.float(), o_hf.float()) < 1e-2 and rel(s, s_hf) < 1e-3, "oracle disagrees with transformers"
    np.savez_compressed(os.path.join(HERE, f"prefill_T{T}.npz"), q=bits(q), k=bits(k), v=bits(v), g=g.numpy(),
                        beta=bits(beta), s0=s0.numpy(), out=bits(o), state=s.numpy())


def decode(seed=100):
    g_ = torch.Generator().manual_seed(seed)
    N, Hk, Hv, D, K = 2, 1, 1, 128, 4
    C = (2 * Hk + Hv) * D
    p = dict(mixed=torch.randn(N, C, generator=g_).to(torch.bfloat16),
             z=torch.randn(N, Hv * D, generator=g_).to(torch.bfloat16),
             a=torch.randn(N, Hv, generator=g_).to(torch.bfloat16),
             b=torch.randn(N, Hv, generator=g_).to(torch.bfloat16),
             conv_state=torch.randn(N, C, K, generator=g_).to(torch.bfloat16),
             conv_weight=(0.5 * torch.randn(C, K, generator=g_)).to(torch.bfloat16),
             A_log=torch.full((Hv,), -2.302585092994046), dt_bias=torch.full((Hv,), 2.0),
             norm_weight=(1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16),
             rec_state=0.02 * torch.randn(N, Hv, D, D, generator=g_))
    conv, rec = p["conv_state"].clone(), p["rec_state"].clone()
    out = O.gdn_decode_core(p["mixed"], p["z"], p["a"], p["b"], conv, p["conv_weight"], p["A_log"],
                            p["dt_bias"], p["norm_weight"], rec, Hk, Hv, D)
    # the recurrent part agrees with transformers' token loop
    st = p["conv_state"].clone()
    qkv = O.elem_conv_update(p["mixed"].unsqueeze(-1), st, p["conv_weight"], None)[:, :, 0]
    beta, gg = O.gdn_gating(p["a"], p["b"], p["A_log"], p["dt_bias"])
    qv, kv, vv = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    _, s_hf = HF.torch_recurrent_gated_delta_rule(qv.reshape(N, 1, 1, D), kv.reshape(N, 1, 1, D),
                                                  vv.reshape(N, 1, 1, D), gg.reshape(N, 1, 1),
                                                  beta.reshape(N, 1, 1), p["rec_state"], True, True)
    assert rel(rec, s_hf) < 1e-6
    np.savez_compressed(os.path.join(HERE, "decode_N2.npz"),
                        **{kk: bits(vv_) for kk, vv_ in p.items()}, out=bits(out), conv_out=bits(conv),
                        rec_out=rec.numpy())


def conv_kat():
    """Integer-valued conv update: every product and sum is exact in bf16."""
    N, C, K = 2, 64, 4
    x = torch.arange(N * C).reshape(N, C, 1).remainder(5).sub(2).to(torch.bfloat16)
    st = torch.arange(N * C * K).reshape(N, C, K).remainder(7).sub(3).to(torch.bfloat16)
    w = torch.arange(C * K).reshape(C, K).remainder(3).sub(1).to(torch.bfloat16)
    st1 = st.clone()
    out = O.elem_conv_update(x, st1, w, None)
    np.savez_compressed(os.path.join(HERE, "conv_kat.npz"), x=bits(x), state=bits(st), w=bits(w),
                        out=bits(out), state_out=bits(st1))


if __name__ == "__main__":
    for T, ws, seed in [(1, True, 1), (63, False, 2), (64, True, 3), (65, True, 4), (130, False, 5)]:
        prefill(T, ws, seed)
    decode()
    conv_kat()
    print("fixtures written to", HERE)
