"""CPU oracle for the Gated DeltaNet (GDN) hot path -- TEST INFRASTRUCTURE ONLY.

This module is the reference restatement used for verification, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The shipped package never imports it and has no
CPU fallback; it fails loudly when its HIP library is missing.

Every function restates, op for op in torch on the CPU, the reference's algorithm for one piece of
the path (citations are ``file:line`` in the reference repository, ``HF:`` = the transformers
``models/qwen3_5/modeling_qwen3_5.py`` that the reference patches; the reference pins transformers
5.5.4, the bodies used here are unchanged in the installed 5.15.0).  Dtype handling follows the
reference exactly: l2norm runs in the input dtype (bf16), the recurrences run in fp32, the conv
update runs in the weight dtype, the gated norm follows HF's cast order.

How each function is pinned (tests/test_oracle.py):
  l2norm                      -- HF ``l2norm`` (library routine): bit-exact on tensors without a
                                 scalar tail in torch's vectorised loop, within one bf16 ulp of the
                                 inverse norm elsewhere (torch double-rounds bf16 rsqrt there).
  unit_lower_inv              -- T (I - X) = I; ``torch.linalg.solve_triangular``; HF's 63-step loop.
  chunk_gated_delta_rule_v2   -- token-by-token recurrence (closed-form equivalence), HF
                                 ``torch_chunk_gated_delta_rule``, padding / split / varlen invariances,
                                 golden fixtures.
  chunk_gated_delta_rule_v1   -- same pins as v2 (equal to v2 up to fp32 rounding).
  recurrent_gated_delta_rule  -- HF ``torch_recurrent_gated_delta_rule`` bit-exact; brute force.
  recurrent_single_step       -- HF token loop at T=1, bit-exact; beta=0, zero-state and exact-write
                                 special cases.
  elem_conv_update            -- integer-valued KAT (exact), brute-force dot products, HF
                                 ``causal_conv1d_update`` within bf16 rounding; state shift exact.
  causal_conv1d_prefill       -- equals repeated decode updates from a zero / given history.
  gated_rmsnorm               -- HF ``Qwen3_5RMSNormGated`` module, bit-exact.
  gdn_gating, expand_key_heads, gdn_decode_core, gdn_prefill_core
                              -- transformers' own ``Qwen3_5GatedDeltaNet.forward`` (the layer the
                                 reference patches) fed the same weights: a fresh prompt, a continued
                                 prompt and cached decode steps, outputs and both states; planted
                                 mistakes (a/b swapped, q/k split swapped, h % r head map, z heads
                                 permuted) are caught.  gdn_gating also against float64.
"""
import torch
import torch.nn.functional as F

__all__ = [
    "l2norm", "small_unit_lower_inv", "unit_lower_inv", "chunk_gated_delta_rule_v1",
    "chunk_gated_delta_rule_v2", "chunk_gated_delta_rule_varlen", "recurrent_gated_delta_rule",
    "recurrent_single_step", "elem_conv_update", "causal_conv1d_update", "causal_conv1d_prefill",
    "gated_rmsnorm", "gdn_gating", "expand_key_heads", "gdn_decode_core", "gdn_prefill_core",
]


def _op(x, dtype):
    """Round an fp32 result once to ``dtype``: the result of one torch elementwise op on a tensor of
    that dtype.  (torch's CPU kernels compute bf16 elementwise ops in fp32 and round once in their
    vectorised body, but double-round some ops such as rsqrt in the scalar tail of the loop, which
    makes the result depend on the element's position by one bf16 ulp; the oracle uses the
    single rounding everywhere.)"""
    return x.to(dtype)


def l2norm(x, dim=-1, eps=1e-6):
    """x * rsqrt(sum(x*x) + eps) with every op rounded to x's dtype, as torch evaluates it on a
    bf16 tensor (products rounded, fp32-accumulated sum rounded, +eps, rsqrt, product).
    src/gdn_chunk_fast.py:17-18, HF:242-245."""
    dt = x.dtype
    xf = x.float()
    sq = _op(xf * xf, dt).float()
    s = _op(sq.sum(dim=dim, keepdim=True), dt).float()
    t = _op(s + eps, dt).float()
    inv = _op(torch.rsqrt(t), dt).float()
    return _op(xf * inv, dt)


def small_unit_lower_inv(X):
    """(I - X)^-1 for strictly lower X by the row recurrence R_i = X_i + sum_j X_ij R_j.
    src/gdn_chunk_fast.py:21-30."""
    n = X.shape[-1]
    R = X.clone()
    for i in range(1, n):
        row = R[..., i, :i].clone()
        sub = R[..., :i, :i].clone()
        R[..., i, :i] = row + (row.unsqueeze(-1) * sub).sum(-2)
    return R + torch.eye(n, dtype=X.dtype, device=X.device)


def unit_lower_inv(X, base=16):
    """Blocked (I - X)^-1: diagonal base x base blocks by the row recurrence, then pairwise merges
    [[A, 0], [B X21 A, B]].  src/gdn_chunk_fast.py:33-62."""
    n = X.shape[-1]
    nb = n // base
    if nb <= 1:
        return small_unit_lower_inv(X)
    diag = torch.stack([X[..., i * base:(i + 1) * base, i * base:(i + 1) * base] for i in range(nb)],
                       dim=-3)
    tdiag = small_unit_lower_inv(diag)
    blocks = [tdiag[..., i, :, :] for i in range(nb)]

    def merge(lo, hi):
        if hi - lo == 1:
            return blocks[lo]
        mid = (lo + hi) // 2
        A = merge(lo, mid)
        B = merge(mid, hi)
        x21 = X[..., mid * base:hi * base, lo * base:mid * base]
        t21 = B @ x21 @ A
        top = torch.cat([A, torch.zeros_like(t21.transpose(-1, -2))], dim=-1)
        bot = torch.cat([t21, B], dim=-1)
        return torch.cat([top, bot], dim=-2)

    return merge(0, nb)


def _prep(query, key, value, g, beta, chunk_size, use_qk_l2norm_in_kernel):
    """Shared prologue of the chunked rule: optional l2norm in the input dtype, fp32 cast,
    [B,T,H,d] -> [B,H,T,d], zero-pad T to a multiple of chunk_size, q *= d^-1/2.
    src/gdn_chunk_fast2.py:13-29 (identical in src/gdn_chunk_fast.py:76-95)."""
    if use_qk_l2norm_in_kernel:
        query = l2norm(query, dim=-1, eps=1e-6)
        key = l2norm(key, dim=-1, eps=1e-6)
    query, key, value, beta, g = [
        x.transpose(1, 2).contiguous().to(torch.float32) for x in (query, key, value, beta, g)]
    L = key.shape[2]
    pad = (chunk_size - L % chunk_size) % chunk_size
    query = F.pad(query, (0, 0, 0, pad))
    key = F.pad(key, (0, 0, 0, pad))
    value = F.pad(value, (0, 0, 0, pad))
    beta = F.pad(beta, (0, pad))
    g = F.pad(g, (0, pad))
    query = query * (1 / (key.shape[-1] ** 0.5))
    return query, key, value, g, beta, L, L + pad


def chunk_gated_delta_rule_v2(query, key, value, g, beta, chunk_size=64, initial_state=None,
                              output_final_state=False, use_qk_l2norm_in_kernel=False, **kwargs):
    """Chunked gated delta rule with all state-independent terms batched over chunks.
    src/gdn_chunk_fast2.py:11-62.  Inputs [B,T,H,d] (q,k already repeated to H_v heads),
    g/beta [B,T,H]; returns (out [B,T,H,d] in query.dtype, final state [B,H,d,d] fp32 | None)."""
    initial_dtype = query.dtype
    query, key, value, g, beta, L, Lp = _prep(query, key, value, g, beta, chunk_size,
                                              use_qk_l2norm_in_kernel)
    B, H, _, dk = key.shape
    dv = value.shape[-1]
    C = chunk_size
    n = Lp // C
    v_beta = value * beta.unsqueeze(-1)
    k_beta = key * beta.unsqueeze(-1)
    query, key, value, k_beta, v_beta = [x.reshape(B, H, n, C, x.shape[-1])
                                         for x in (query, key, value, k_beta, v_beta)]
    g = g.reshape(B, H, n, C).cumsum(dim=-1)
    tri_strict = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=0)
    tri_incl = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=1)
    decay = (g.unsqueeze(-1) - g.unsqueeze(-2)).tril().exp().float().tril()
    X = -((k_beta @ key.transpose(-1, -2)) * decay).masked_fill(tri_strict, 0)
    attn = unit_lower_inv(X)
    V = attn @ v_beta
    Kc = attn @ (k_beta * g.exp().unsqueeze(-1))
    QK = ((query @ key.transpose(-1, -2)) * decay).masked_fill(tri_incl, 0)
    Qg = query * g.exp().unsqueeze(-1)
    glast = g[..., -1]
    Gl = glast.exp()
    Kd = (key * (glast.unsqueeze(-1) - g).exp().unsqueeze(-1)).transpose(-1, -2)
    S = (torch.zeros(B, H, dk, dv, dtype=torch.float32) if initial_state is None
         else initial_state.to(torch.float32))
    outs = [torch.zeros(B, H, 0, C, dv)] if n == 0 else []   # empty sequence: no chunks
    for i in range(n):
        vn = V[:, :, i] - Kc[:, :, i] @ S
        outs.append(Qg[:, :, i] @ S + QK[:, :, i] @ vn)
        S = S * Gl[:, :, i, None, None] + Kd[:, :, i] @ vn
    core = torch.stack(outs, dim=2).reshape(B, H, Lp, dv)[:, :, :L]
    return core.transpose(1, 2).contiguous().to(initial_dtype), (S if output_final_state else None)


def chunk_gated_delta_rule_v1(query, key, value, g, beta, chunk_size=64, initial_state=None,
                              output_final_state=False, use_qk_l2norm_in_kernel=False, **kwargs):
    """Chunked gated delta rule with the per-chunk products inside the loop.
    src/gdn_chunk_fast.py:65-142."""
    initial_dtype = query.dtype
    query, key, value, g, beta, L, Lp = _prep(query, key, value, g, beta, chunk_size,
                                              use_qk_l2norm_in_kernel)
    B, H, _, dk = key.shape
    dv = value.shape[-1]
    C = chunk_size
    v_beta = value * beta.unsqueeze(-1)
    k_beta = key * beta.unsqueeze(-1)
    query, key, value, k_beta, v_beta = [x.reshape(B, H, -1, C, x.shape[-1])
                                         for x in (query, key, value, k_beta, v_beta)]
    g = g.reshape(B, H, -1, C).cumsum(dim=-1)
    strict_upper_or_diag = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=0)
    decay_mask = ((g.unsqueeze(-1) - g.unsqueeze(-2)).tril().exp().float()).tril()
    X = -((k_beta @ key.transpose(-1, -2)) * decay_mask).masked_fill(strict_upper_or_diag, 0)
    attn = unit_lower_inv(X)
    value = attn @ v_beta
    k_cumdecay = attn @ (k_beta * g.exp().unsqueeze(-1))
    S = (torch.zeros(B, H, dk, dv, dtype=torch.float32) if initial_state is None
         else initial_state.to(torch.float32))
    mask = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=1)
    outs = []
    for i in range(Lp // C):
        q_i, k_i, v_i = query[:, :, i], key[:, :, i], value[:, :, i]
        attn_i = (q_i @ k_i.transpose(-1, -2) * decay_mask[:, :, i]).masked_fill(mask, 0)
        v_new = v_i - k_cumdecay[:, :, i] @ S
        attn_inter = (q_i * g[:, :, i, :, None].exp()) @ S
        outs.append(attn_inter + attn_i @ v_new)
        S = (S * g[:, :, i, -1, None, None].exp()
             + (k_i * (g[:, :, i, -1, None] - g[:, :, i]).exp()[..., None]).transpose(-1, -2) @ v_new)
    core = torch.stack(outs, dim=2).reshape(B, H, Lp, dv)[:, :, :L]
    return core.transpose(1, 2).contiguous().to(initial_dtype), (S if output_final_state else None)


def chunk_gated_delta_rule_varlen(query, key, value, g, beta, cu_seqlens, chunk_size=64,
                                  initial_state=None, output_final_state=False,
                                  use_qk_l2norm_in_kernel=False):
    """Packed varlen prefill [1, sum T, H, d] with int cu_seqlens [n_seq+1]: the reference has no
    varlen kernel, so this is its per-sequence loop (src/cb_tp.py:196-261 runs one sequence per call).
    initial_state [n_seq,H,dk,dv] or None.  Returns (out [1,sumT,H,dv], final [n_seq,H,dk,dv] | None)."""
    cu = [int(c) for c in cu_seqlens]
    outs, finals = [], []
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        init = None if initial_state is None else initial_state[s:s + 1]
        o, st = chunk_gated_delta_rule_v2(query[:, a:b], key[:, a:b], value[:, a:b], g[:, a:b],
                                          beta[:, a:b], chunk_size, init, True,
                                          use_qk_l2norm_in_kernel)
        outs.append(o)
        finals.append(st)
    out = torch.cat(outs, dim=1)
    return out, (torch.cat(finals, dim=0) if output_final_state else None)


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state, output_final_state,
                               use_qk_l2norm_in_kernel=False, **kwargs):
    """Token-by-token gated delta rule (HF:331-384, the T>1 branch of src/recurrent_single_step.py:10-13)."""
    initial_dtype = query.dtype
    if use_qk_l2norm_in_kernel:
        query = l2norm(query, dim=-1, eps=1e-6)
        key = l2norm(key, dim=-1, eps=1e-6)
    query, key, value, beta, g = [x.transpose(1, 2).contiguous().to(torch.float32)
                                  for x in (query, key, value, beta, g)]
    B, H, T, dk = key.shape
    dv = value.shape[-1]
    query = query * (1 / (query.shape[-1] ** 0.5))
    out = torch.zeros(B, H, T, dv, dtype=torch.float32)
    S = (torch.zeros(B, H, dk, dv, dtype=torch.float32) if initial_state is None
         else initial_state.to(torch.float32))
    for i in range(T):
        q_t, k_t, v_t = query[:, :, i], key[:, :, i], value[:, :, i]
        g_t = g[:, :, i].exp().unsqueeze(-1).unsqueeze(-1)
        beta_t = beta[:, :, i].unsqueeze(-1)
        S = S * g_t
        kv_mem = (S * k_t.unsqueeze(-1)).sum(dim=-2)
        delta = (v_t - kv_mem) * beta_t
        S = S + k_t.unsqueeze(-1) * delta.unsqueeze(-2)
        out[:, :, i] = (S * q_t.unsqueeze(-1)).sum(dim=-2)
    return out.transpose(1, 2).contiguous().to(initial_dtype), (S if output_final_state else None)


def recurrent_single_step(query, key, value, g, beta, initial_state, output_final_state,
                          use_qk_l2norm_in_kernel=False):
    """One-token gated delta rule in fp32.  src/recurrent_single_step.py:8-32.
    q,k,v [N,1,H,d], g [N,1,H] fp32, beta [N,1,H], state [N,H,dk,dv]; returns a NEW state."""
    if query.shape[1] != 1:
        return recurrent_gated_delta_rule(query, key, value, g, beta, initial_state,
                                          output_final_state, use_qk_l2norm_in_kernel)
    initial_dtype = query.dtype
    if use_qk_l2norm_in_kernel:
        query = l2norm(query, dim=-1, eps=1e-6)
        key = l2norm(key, dim=-1, eps=1e-6)
    q, k, v, beta, g = [x[:, 0].contiguous().to(torch.float32) for x in (query, key, value, beta, g)]
    q = q * (1 / (query.shape[-1] ** 0.5))
    state = (torch.zeros((*k.shape, v.shape[-1]), dtype=v.dtype) if initial_state is None
             else initial_state.to(v))
    state = state * g.exp().unsqueeze(-1).unsqueeze(-1)
    memory = (state * k.unsqueeze(-1)).sum(dim=-2)
    delta = (v - memory) * beta.unsqueeze(-1)
    state = state + k.unsqueeze(-1) * delta.unsqueeze(-2)
    output = (state * q.unsqueeze(-1)).sum(dim=-2)
    return output.unsqueeze(1).to(initial_dtype), (state if output_final_state else None)


def elem_conv_update(x, state, weight, bias):
    """Decode depthwise causal conv by mul + sum over the K-window; shifts ``state`` in place.
    x [n,C,1], state [n,C,K], weight [C,K], bias [C] | None -> silu(conv) [n,C,1].
    src/cb_engine.py:43-51."""
    hs = torch.cat([state, x], dim=-1).to(weight.dtype)
    state.copy_(hs[:, :, -state.shape[-1]:])
    win = hs[:, :, -weight.shape[-1]:]
    out = (win * weight).sum(-1, keepdim=True)
    if bias is not None:
        out = out + bias.view(1, -1, 1)
    return _op(F.silu(out.float()), out.dtype).to(x.dtype)


def causal_conv1d_update(hidden_states, conv_state, weight, bias=None, activation=None):
    """HF's decode conv through F.conv1d (HF:200-217); same contract as elem_conv_update."""
    _, hidden_size, seq_len = hidden_states.shape
    state_len = conv_state.shape[-1]
    hs = torch.cat([conv_state, hidden_states], dim=-1).to(weight.dtype)
    conv_state.copy_(hs[:, :, -state_len:])
    out = F.conv1d(hs, weight.unsqueeze(1), bias, padding=0, groups=hidden_size)[:, :, -seq_len:]
    if activation is not None:
        out = F.silu(out)
    return out.to(hidden_states.dtype)


def causal_conv1d_prefill(x, weight, bias=None, history=None):
    """Depthwise causal conv + SiLU over a prompt, and the decode conv state it leaves.
    x [1,C,L]; history None (fresh prompt: zero history, F.conv1d padding K-1, src/cb_tp.py:163-164)
    or [1,C,K] (the previous K inputs, src/cb_tp.py:236-244).  Returns (out [1,C,L] in x.dtype,
    new_state [1,C,K] = last K inputs, left zero-padded, src/cb_tp.py:158-162 and :260)."""
    C, K = weight.shape
    L = x.shape[-1]
    if L == 0:  # empty prompt: no outputs, the state keeps the history (or zeros)
        state = torch.zeros(x.shape[0], C, K, dtype=x.dtype) if history is None else history.to(x.dtype)
        return x.clone(), state.contiguous()
    if history is None:
        conv = F.conv1d(x, weight.unsqueeze(1), bias, padding=K - 1, groups=C)[:, :, :L]
        state = x[:, :, -K:] if L >= K else F.pad(x, (K - L, 0))
    else:
        full = torch.cat([history.to(x.dtype), x], dim=-1)
        conv = F.conv1d(full[:, :, 1:], weight.unsqueeze(1), bias, groups=C)
        state = full[:, :, -K:]
    out = _op(F.silu(conv.float()), conv.dtype)
    return out.to(x.dtype), state.contiguous()


def gated_rmsnorm(hidden_states, gate, weight, eps=1e-6):
    """silu(gate) * (rmsnorm(x) cast to x.dtype * weight), HF order.  HF:175-184
    (the reference's src/cb_engine.py:65-67 runs the closed npu_rms_norm + npu_swiglu instead)."""
    input_dtype = hidden_states.dtype
    h = hidden_states.to(torch.float32)
    variance = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(variance + eps)
    h = weight * h.to(input_dtype)
    h = h * F.silu(gate.to(torch.float32))
    return h.to(input_dtype)


def gdn_gating(a, b, A_log, dt_bias):
    """beta = sigmoid(b) (input dtype), g = -exp(A_log) * softplus(a + dt_bias) in fp32.
    src/cb_engine.py:337-338 (HF:497-498)."""
    beta = _op(b.float().sigmoid(), b.dtype)
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias)
    return beta, g


def expand_key_heads(x, r):
    """[.., H_k, d] -> [.., H_k * r, d] with value head h reading key head h // r
    (``repeat_interleave(r, dim=2)``, src/cb_engine.py:339-342, HF:499-502)."""
    return x.repeat_interleave(r, dim=2) if r > 1 else x


def gdn_decode_core(mixed_qkv, z, a, b, conv_state, conv_weight, A_log, dt_bias, norm_weight,
                    rec_state, num_k_heads, num_v_heads, head_dim, eps=1e-6, conv_bias=None):
    """The GDN decode layer between the input projections and out_proj:
    elem conv update -> split q/k/v -> gating -> repeat_interleave -> recurrent step -> state write
    -> gated norm.  src/cb_engine.py:318-351 with ELEM_CONV (src/cb_engine.py:326-328).
    mixed_qkv [N,C] (pre-conv), z [N,H_v*d], a,b [N,H_v]; conv_state [N,C,K] and rec_state
    [N,H_v,d,d] fp32 are updated in place.  Returns the normed core [N, H_v*d] in mixed's dtype."""
    n = mixed_qkv.shape[0]
    kd = num_k_heads * head_dim
    mixed = elem_conv_update(mixed_qkv.unsqueeze(-1), conv_state, conv_weight, conv_bias)
    mixed = mixed.transpose(1, 2)
    query, key, value = torch.split(mixed, [kd, kd, num_v_heads * head_dim], dim=-1)
    query = query.reshape(n, 1, -1, head_dim)
    key = key.reshape(n, 1, -1, head_dim)
    value = value.reshape(n, 1, -1, head_dim)
    beta, g = gdn_gating(a.reshape(n, 1, -1), b.reshape(n, 1, -1), A_log, dt_bias)
    r = num_v_heads // num_k_heads
    query, key = expand_key_heads(query, r), expand_key_heads(key, r)
    core, new_rs = recurrent_single_step(query, key, value, g, beta, rec_state, True, True)
    rec_state.copy_(new_rs.to(rec_state.dtype))
    core = gated_rmsnorm(core.reshape(-1, head_dim), z.reshape(-1, head_dim), norm_weight, eps)
    return core.reshape(n, -1)


def gdn_prefill_core(mixed_qkv, z, a, b, conv_weight, A_log, dt_bias, norm_weight, num_k_heads,
                     num_v_heads, head_dim, cu_seqlens=None, conv_history=None, initial_state=None,
                     eps=1e-6, chunk_size=64, conv_bias=None):
    """The GDN prefill layer between the input projections and out_proj, for one or more packed
    sequences: conv prefill + SiLU (fresh or continued history) -> split -> gating -> repeat ->
    chunked rule (v2) -> gated norm.  src/cb_tp.py:153-181 (fresh prompt) and :230-263 (continuation).
    mixed_qkv [T_total, C], z [T_total, H_v*d], a,b [T_total, H_v]; cu_seqlens [n_seq+1] or None
    (one sequence); conv_history [n_seq,C,K] | None; initial_state [n_seq,H_v,d,d] | None.
    Returns (core [T_total, H_v*d], conv_state [n_seq,C,K], rec_state [n_seq,H_v,d,d] fp32)."""
    T = mixed_qkv.shape[0]
    cu = [0, T] if cu_seqlens is None else [int(c) for c in cu_seqlens]
    kd = num_k_heads * head_dim
    r = num_v_heads // num_k_heads
    cores, convs, recs = [], [], []
    for s in range(len(cu) - 1):
        lo, hi = cu[s], cu[s + 1]
        L = hi - lo
        x = mixed_qkv[lo:hi].t().unsqueeze(0)                       # [1,C,L]
        hist = None if conv_history is None else conv_history[s:s + 1]
        mixed, cstate = causal_conv1d_prefill(x, conv_weight, conv_bias, hist)
        mixed = mixed.transpose(1, 2)
        query, key, value = torch.split(mixed, [kd, kd, num_v_heads * head_dim], dim=-1)
        query = query.reshape(1, L, num_k_heads, head_dim)
        key = key.reshape(1, L, num_k_heads, head_dim)
        value = value.reshape(1, L, num_v_heads, head_dim)
        beta, g = gdn_gating(a[lo:hi].unsqueeze(0), b[lo:hi].unsqueeze(0), A_log, dt_bias)
        query, key = expand_key_heads(query, r), expand_key_heads(key, r)
        init = None if initial_state is None else initial_state[s:s + 1]
        core, last = chunk_gated_delta_rule_v2(query, key, value, g, beta, chunk_size, init, True, True)
        core = gated_rmsnorm(core.reshape(-1, head_dim), z[lo:hi].reshape(-1, head_dim),
                             norm_weight, eps)
        cores.append(core.reshape(L, num_v_heads * head_dim))
        convs.append(cstate.to(mixed_qkv.dtype))
        recs.append(last)
    return torch.cat(cores, 0), torch.cat(convs, 0), torch.cat(recs, 0)
