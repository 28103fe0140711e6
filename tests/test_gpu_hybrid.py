"""GPU tests of the whole-layer decode path: a GDN layer with its projections against an fp32
composition around the oracle (src/cb_engine.py:318-352), the full-attention layer against a
per-slot fp32 reference, and the graph-captured hybrid step (src/cb_engine.py:123-187) against
eager steps."""
import importlib

import pytest
import torch

from conftest import PKG_NAME, rel_l2

OUT_TOL = 1e-2


def rms_norm(x, w, eps):
    """Qwen3_5RMSNorm (HF modeling_qwen3_5.py): fp32 x * rsqrt(mean(x^2) + eps) * (1 + w), cast back."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (y * (1.0 + w.float())).to(x.dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _hybrid(gdn):
    from importlib import import_module
    return import_module(PKG_NAME + ".hybrid_decode")


def _small_cfg(hd_mod):
    return hd_mod.HybridConfig(hidden=256, layers=4, full_every=4, gdn_k_heads=2, gdn_v_heads=4, gdn_head=128,
                               conv_k=4, attn_heads=4, kv_heads=2, attn_head=64, mlp=512, vocab=128)


@pytest.mark.gpu
def test_gdn_layer_with_projections_vs_oracle(gdn, oracle, dev):
    """in_proj (one GEMM) -> fused HIP core -> out_proj equals the fp32 composition of the same
    weights around the oracle's decode core; the layer's states match too."""
    hd = _hybrid(gdn)
    cfg = _small_cfg(hd)
    model = hd.HybridDecoder(cfg, 3, [5, 17, 9], 4, dev, seed=40, keep_plain=True)
    L = model.layers[0]
    g_ = torch.Generator().manual_seed(41)
    x = torch.randn(3, cfg.hidden, generator=g_).to(torch.bfloat16)
    conv0, rec0 = model.slots.conv[0].cpu(), model.slots.rec[0].cpu()
    out = model.gdn(0, L, x.to(dev)).cpu()
    Hv, D, C = cfg.gdn_v_heads, cfg.gdn_head, cfg.conv_dim
    # the layer's own projection (its packed-weight HIP product, deterministic) against an fp32 GEMM,
    # then fed to the oracle: the conv state (the pre-conv inputs shifted in) is exact
    cb = importlib.import_module(PKG_NAME + ".cb_engine")
    proj = cb.decode_linear(x.to(dev), L.in_proj_p).cpu()
    assert rel_l2(proj, x.float() @ L.in_proj.cpu().float().t()) <= 1e-2
    mixed, z = proj[:, :C], proj[:, C:C + Hv * D]
    b, a = proj[:, C + Hv * D:C + Hv * D + Hv], proj[:, C + Hv * D + Hv:]
    conv_ref, rec_ref = conv0.clone(), rec0.clone()
    core = oracle.gdn_decode_core(mixed, z, a, b, conv_ref, L.conv_w.cpu(), L.A_log.cpu(), L.dt_bias.cpu(),
                                  L.norm_w.cpu(), rec_ref, cfg.gdn_k_heads, Hv, D, cfg.eps)
    ref = core.float() @ L.out.cpu().float().t()
    assert rel_l2(out, ref) <= OUT_TOL
    assert rel_l2(model.slots.rec[0], rec_ref) <= 1e-3
    assert torch.equal(model.slots.conv[0].cpu(), conv_ref)


@pytest.mark.gpu
def test_attention_layer_vs_fp32_reference(gdn, dev):
    """GQA decode attention (gated q, q/k RMSNorm, partial rotary, KV cache at each slot's position)
    against a per-slot fp32 loop over the same cache."""
    hd = _hybrid(gdn)
    cfg = _small_cfg(hd)
    ctx = [5, 17, 9]
    model = hd.HybridDecoder(cfg, 3, ctx, 4, dev, seed=42, keep_plain=True)
    L = model.layers[3]
    g_ = torch.Generator().manual_seed(43)
    x = torch.randn(3, cfg.hidden, generator=g_).to(torch.bfloat16)
    out = model.attention(L, x.to(dev)).cpu().float()
    nh, kv, hdim = cfg.attn_heads, cfg.kv_heads, cfg.attn_head
    rd = int(hdim * cfg.rotary_frac)
    kt, vc = L.kt.cpu().float(), L.v.cpu().float()   # the cache after the layer wrote this token
    proj = (x.float() @ L.qkv.cpu().float().t())
    ref = torch.zeros(3, cfg.hidden)
    for n in range(3):
        p = ctx[n]
        qg = proj[n, :nh * hdim * 2].reshape(nh, 2 * hdim)
        q, gate = qg[:, :hdim], qg[:, hdim:].reshape(-1)
        q = rms_norm(q, L.q_norm.cpu(), cfg.eps)
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, rd, 2).float() / rd))
        emb = torch.cat((p * inv, p * inv))
        qr = q[:, :rd] * emb.cos() + rotate_half(q[:, :rd]) * emb.sin()
        q = torch.cat((qr, q[:, rd:]), dim=-1)
        o = torch.zeros(nh, hdim)
        for h in range(nh):
            j = h // (nh // kv)
            s = (q[h] @ kt[n, j, :, :p + 1]) * hdim ** -0.5
            o[h] = torch.softmax(s, -1) @ vc[n, j, :p + 1, :]
        ref[n] = (o.reshape(-1) * torch.sigmoid(gate)) @ L.o.cpu().float().t()
    assert rel_l2(out, ref) <= OUT_TOL
    # the new key / value landed at each slot's position and nowhere else
    kproj = proj[:, nh * hdim * 2:nh * hdim * 2 + kv * hdim].reshape(3, kv, hdim)
    for n in range(3):
        k_ref = rms_norm(kproj[n], L.k_norm.cpu(), cfg.eps)
        assert rel_l2(kt[n, :, rd:, ctx[n]], k_ref[:, rd:]) <= 1e-2


def _attn_reference(proj, pos, qn, kn, inv_freq, kt, vc, nh, kv, hd, rd, eps):
    """Per-slot fp32 loop of HF Qwen3_5Attention at decode on the CPU; updates kt / vc in place."""
    N = proj.shape[0]
    out = torch.zeros(N, nh * hd)
    for n in range(N):
        p = int(pos[n])
        emb = torch.cat((p * inv_freq, p * inv_freq))
        cos, sin = emb.cos(), emb.sin()

        def rope(t):
            tr = t[..., :rd].float()
            return torch.cat(((tr * cos + rotate_half(tr) * sin).to(t.dtype), t[..., rd:]), dim=-1)

        qg = proj[n, :nh * 2 * hd].reshape(nh, 2 * hd)
        q = rope(rms_norm(qg[:, :hd], qn, eps))
        gate = qg[:, hd:].reshape(-1)
        k = rope(rms_norm(proj[n, 2 * nh * hd:(2 * nh + kv) * hd].reshape(kv, hd), kn, eps))
        v = proj[n, (2 * nh + kv) * hd:(2 * nh + 2 * kv) * hd].reshape(kv, hd)
        kt[n, :, :, p] = k
        vc[n, :, p, :] = v
        o = torch.zeros(nh, hd)
        for h in range(nh):
            j = h // (nh // kv)
            s = (q[h].float() @ kt[n, j, :, :p + 1].float()) * hd ** -0.5
            o[h] = torch.softmax(s, -1) @ vc[n, j, :p + 1, :].float()
        out[n] = (o.reshape(-1).to(torch.bfloat16) * torch.sigmoid(gate)).float()
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("nh,kv,hd,pos,T", [
    (24, 4, 256, [0, 255, 256, 1300], 1304),   # 27B shape; split edges at 256 positions
    (4, 2, 64, [5, 17, 9], 24),
    (8, 1, 128, [700, 3], 704),
    (2, 2, 128, [511, 515], 516),
])
def test_gqa_decode_attention_vs_fp32(gdn, dev, nh, kv, hd, pos, T):
    """The three-launch decode attention (q/k norm, partial rotary, cache writes at each slot's
    position, split softmax attention, gate) against a per-slot fp32 loop; the caches hold the new
    key and value at each position and are unchanged elsewhere."""
    from importlib import import_module
    cb = import_module(PKG_NAME + ".cb_engine")
    N, rd, eps = len(pos), hd // 4, 1e-6
    g_ = torch.Generator().manual_seed(hd + nh + T)
    bf = torch.bfloat16
    proj = torch.randn(N, (2 * nh + 2 * kv) * hd, generator=g_).to(bf)
    qn = (0.1 * torch.randn(hd, generator=g_)).to(bf)
    kn = (0.1 * torch.randn(hd, generator=g_)).to(bf)
    inv = 1.0 / (10000.0 ** (torch.arange(0, rd, 2).float() / rd))
    kt = torch.randn(N, kv, hd, T, generator=g_).to(bf)
    vc = torch.randn(N, kv, T, hd, generator=g_).to(bf)
    pos_t = torch.tensor(pos, dtype=torch.int64)
    kt_d, vc_d = kt.to(dev), vc.to(dev)
    out = cb.gqa_decode_attention(proj.to(dev), pos_t.to(dev), qn.to(dev), kn.to(dev), inv.to(dev), kt_d, vc_d,
                                  nh, kv, hd, rd, eps).cpu().float()
    ref = _attn_reference(proj, pos_t, qn, kn, inv, kt, vc, nh, kv, hd, rd, eps)
    assert rel_l2(out, ref) <= OUT_TOL
    kt_g, vc_g = kt_d.cpu(), vc_d.cpu()
    assert torch.equal(vc_g, vc)                       # values copied exactly, nothing else touched
    for n, p in enumerate(pos):
        assert rel_l2(kt_g[n, :, :, p], kt[n, :, :, p]) <= 1e-2
        kt_g[n, :, :, p] = kt[n, :, :, p]
    assert torch.equal(kt_g, kt)


@pytest.mark.gpu
@pytest.mark.parametrize("nh,kv,hd,H", [(4, 2, 64, 512), (24, 4, 256, 5120)])
def test_gqa_decode_attention_from_partials(gdn, dev, nh, kv, hd, H):
    """The attention fed the q|gate|k|v projection's split-K partials gives exactly what it gives on the
    reduced projection: the same output and the same cache writes."""
    from importlib import import_module
    cb = import_module(PKG_NAME + ".cb_engine")
    g_ = torch.Generator().manual_seed(50)
    bf = torch.bfloat16
    N, T, rd = 16, 520, hd // 4
    x = torch.randn(N, H, generator=g_).to(bf).to(dev)
    w = cb.PackedWeight((0.05 * torch.randn((2 * nh + 2 * kv) * hd, H, generator=g_)).to(bf).to(dev))
    qn = (0.1 * torch.randn(hd, generator=g_)).to(bf).to(dev)
    kn = (0.1 * torch.randn(hd, generator=g_)).to(bf).to(dev)
    inv = (1.0 / (10000.0 ** (torch.arange(0, rd, 2).float() / rd))).to(dev)
    kt = torch.randn(N, kv, hd, T, generator=g_).to(bf).to(dev)
    vc = torch.randn(N, kv, T, hd, generator=g_).to(bf).to(dev)
    pos = torch.randint(0, T, (N,), generator=g_).to(dev)
    p = cb.decode_linear_partial(x, w)
    assert p.splits > 1
    kt1, vc1, kt2, vc2 = kt.clone(), vc.clone(), kt.clone(), vc.clone()
    o1 = cb.gqa_decode_attention(cb.decode_linear(x, w), pos, qn, kn, inv, kt1, vc1, nh, kv, hd, rd)
    o2 = cb.gqa_decode_attention(p, pos, qn, kn, inv, kt2, vc2, nh, kv, hd, rd)
    assert torch.equal(o1, o2) and torch.equal(kt1, kt2) and torch.equal(vc1, vc2)


@pytest.mark.gpu
def test_gqa_decode_attention_negative_position(gdn, dev):
    """A slot at position -1 attends to nothing: zero output and no cache write; the other slots are
    unaffected."""
    from importlib import import_module
    cb = import_module(PKG_NAME + ".cb_engine")
    nh, kv, hd, T, rd, eps = 4, 2, 64, 16, 16, 1e-6
    g_ = torch.Generator().manual_seed(49)
    bf = torch.bfloat16
    proj = torch.randn(2, (2 * nh + 2 * kv) * hd, generator=g_).to(bf)
    qn = (0.1 * torch.randn(hd, generator=g_)).to(bf)
    kn = (0.1 * torch.randn(hd, generator=g_)).to(bf)
    inv = 1.0 / (10000.0 ** (torch.arange(0, rd, 2).float() / rd))
    kt = torch.randn(2, kv, hd, T, generator=g_).to(bf)
    vc = torch.randn(2, kv, T, hd, generator=g_).to(bf)
    kt_d, vc_d = kt.to(dev), vc.to(dev)
    out = cb.gqa_decode_attention(proj.to(dev), torch.tensor([-1, 5], device=dev), qn.to(dev), kn.to(dev),
                                  inv.to(dev), kt_d, vc_d, nh, kv, hd, rd, eps).cpu().float()
    assert torch.equal(out[0], torch.zeros(nh * hd))
    assert torch.equal(kt_d[0].cpu(), kt[0]) and torch.equal(vc_d[0].cpu(), vc[0])
    ref = _attn_reference(proj[1:], torch.tensor([5]), qn, kn, inv, kt[1:].clone(), vc[1:].clone(), nh, kv, hd, rd,
                          eps)
    assert rel_l2(out[1:], ref) <= OUT_TOL


@pytest.mark.gpu
def test_hybrid_graph_replay_matches_eager(gdn, dev):
    """Three replays of the captured 4-layer hybrid step give the eager steps' logits and states."""
    hd = _hybrid(gdn)
    cfg = _small_cfg(hd)
    ctx = [5, 17, 9]
    eager = hd.HybridDecoder(cfg, 3, ctx, 8, dev, seed=44)
    graphed = hd.HybridDecoder(cfg, 3, ctx, 8, dev, seed=44)
    g_ = torch.Generator().manual_seed(45)
    inp = torch.randn(3, cfg.hidden, generator=g_).to(torch.bfloat16).to(dev)
    graph = hd.HybridDecodeGraph(graphed, inp)        # runs one eager warm-up step
    eager.step(inp)
    for _ in range(3):
        out_g = graph.replay().clone()
        out_e = eager.step(inp)
        torch.cuda.synchronize()
        assert rel_l2(out_g, out_e) <= 1e-3
        for i in eager.slots.rec:
            assert rel_l2(graphed.slots.rec[i], eager.slots.rec[i]) <= 1e-5
            assert torch.equal(graphed.slots.conv[i], eager.slots.conv[i])
        assert torch.equal(graphed.pos, eager.pos)


@pytest.mark.gpu
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("M,N,K", [(16, 16480, 5120), (16, 5120, 6144), (3, 98, 256), (16, 1000, 17408),
                                   (1, 4096, 1024)])
def test_decode_linear_vs_fp32(gdn, dev, M, N, K, packed):
    """The decode-projection kernel, on plain and on packed weights (split and unsplit K, row tails,
    N not a multiple of 4 or 16), against an fp32 product of the same bf16 operands."""
    from importlib import import_module
    cb = import_module(PKG_NAME + ".cb_engine")
    g_ = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g_).to(torch.bfloat16)
    w = (0.02 * torch.randn(N, K, generator=g_)).to(torch.bfloat16)
    wd = w.to(dev)
    out = cb.decode_linear(x.to(dev), cb.PackedWeight(wd) if packed else wd).cpu()
    ref = x.float() @ w.float().t()
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    # fp32 accumulation, one bf16 rounding: within a bf16 ulp of each element plus summation order
    assert ((out.float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-3).all()


@pytest.mark.gpu
@pytest.mark.parametrize("H", [5120, 4096, 5121, 12288])
def test_add_rms_norm_vs_torch(gdn, dev, H):
    """Fused residual add + Qwen3_5RMSNorm against the torch formula (residual rounded to bf16 first);
    H = 4096 / 5120: the vector kernel (2 / 4 pieces per thread), 5121 and 12288: the element loop."""
    from importlib import import_module
    cb = import_module(PKG_NAME + ".cb_engine")
    hd = _hybrid(gdn)
    g_ = torch.Generator().manual_seed(46)
    h = torch.randn(5, H, generator=g_).to(torch.bfloat16)
    d = torch.randn(5, H, generator=g_).to(torch.bfloat16)
    w = (0.02 * torch.randn(H, generator=g_)).to(torch.bfloat16)
    h2, x = cb.add_rms_norm(h.to(dev), d.to(dev), w.to(dev))
    assert torch.equal(h2.cpu(), h + d)
    x_ref = rms_norm(h + d, w, 1e-6)
    assert ((x.cpu().float() - x_ref.float()).abs() <= x_ref.float().abs() * 2 ** -7 + 1e-6).all()
    h3, x0 = cb.add_rms_norm(h.to(dev), None, w.to(dev))
    assert torch.equal(h3.cpu(), h)
    assert rel_l2(x0, rms_norm(h, w, 1e-6)) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(5120, 6144), (512, 1024), (34816, 5120)])
def test_split_k_partials_feed_norm_and_swiglu(gdn, dev, N, K):
    """The split-K partial sums of a projection, reduced by their consumers, give exactly the reduced
    projection's values: residual add + norm from partials == from the bf16 output, SwiGLU from the
    gate_up partials == bf16(bf16(silu(g)) * u) of the reduced output, with torch's CPU SiLU (fp32,
    one rounding: the kernel's bf16 SiLU is that function for every bf16 input)."""
    from importlib import import_module
    cb = import_module(PKG_NAME + ".cb_engine")
    g_ = torch.Generator().manual_seed(47)
    M = 16
    x = torch.randn(M, K, generator=g_).to(torch.bfloat16).to(dev)
    w = cb.PackedWeight((0.02 * torch.randn(N, K, generator=g_)).to(torch.bfloat16).to(dev))
    y = cb.decode_linear(x, w)
    p = cb.decode_linear_partial(x, w)
    assert torch.equal(p.to_bf16(), y), "partials must reduce to the projection's output"
    if N <= 8192:
        h = torch.randn(M, N, generator=g_).to(torch.bfloat16).to(dev)
        nw = (0.02 * torch.randn(N, generator=g_)).to(torch.bfloat16).to(dev)
        h_ref, x_ref = cb.add_rms_norm(h, y, nw)
        h_p, x_p = cb.add_rms_norm(h, p, nw)
        assert torch.equal(h_p, h_ref) and torch.equal(x_p, x_ref)
    if N % 16 == 0:
        m = N // 2
        act = cb.swiglu(p)
        yc = y.cpu()
        silu = torch.nn.functional.silu(yc[:, :m].float()).to(torch.bfloat16)
        assert torch.equal(act.cpu(), (silu.float() * yc[:, m:].float()).to(torch.bfloat16))
        ref = cb.swiglu(y)  # torch's GPU SiLU: within one bf16 ulp
        assert ((act.float() - ref.float()).abs() <= ref.float().abs() * 2 ** -7).all()
