"""GDN pieces of the continuous-batching engine on the HIP library.

Mirrors the hot-path parts of the reference engine (src/cb_engine.py):
  * ``elem_conv_update``      -- src/cb_engine.py:43-51 (decode conv, state shifted in place)
  * ``causal_conv1d_update``  -- HF name of the same update (HF modeling_qwen3_5.py:200-217)
  * ``gated_rmsnorm`` / ``fused_gated_rmsnorm`` -- src/cb_engine.py:65-67 (HF formula, HF:175-184)
  * ``patch_model``           -- src/cb_engine.py:54-77
  * ``gdn_decode_core``       -- the fused middle of CBEngine._gdn (src/cb_engine.py:325-351)
  * ``GDNSlots`` / ``gdn_decode_layer`` / ``GDNDecodeGraph`` -- the slot-state layout
    (src/cb_engine.py:103-113), the decode layer (src/cb_engine.py:318-352) and the graph-captured
    decode step (src/cb_engine.py:123-187) restricted to the GDN layers.
Layouts are the reference's: conv state [N, C, K] bf16, recurrent state [N, H_v, d_k, d_v] fp32.
"""
import torch

from . import _lib
from .recurrent_single_step import recurrent_single_step

# The decode conv is always the mul+sum window form (the reference's --elem-conv, cb_run.py:98,160).
ELEM_CONV = True


def _row_view(x2d):
    """[rows, C] with unit inner stride; returns (tensor, row stride)."""
    if x2d.stride(-1) != 1:
        x2d = x2d.contiguous()
    return x2d, x2d.stride(0)


def elem_conv_update(x, state, weight, bias):
    """x [n,C,1] bf16, state [n,C,K] bf16 (updated in place), weight [C,K] bf16, bias [C] | None.
    Returns silu(conv) [n,C,1] in x.dtype.  src/cb_engine.py:43-51."""
    _lib.require_cuda(x, state, weight, bias)
    n, C, T = x.shape
    if T != 1:
        raise ValueError("elem_conv_update: one token per call (x [n,C,1])")
    K = weight.shape[-1]
    if tuple(state.shape) != (n, C, K) or tuple(weight.shape) != (C, K):
        raise ValueError(f"elem_conv_update: state {tuple(state.shape)} / weight {tuple(weight.shape)} "
                         f"do not match x {tuple(x.shape)}")
    if not (x.dtype == state.dtype == weight.dtype == torch.bfloat16):
        raise TypeError("elem_conv_update: x, state and weight must be bfloat16")
    if not state.is_contiguous():
        raise ValueError("elem_conv_update: state must be contiguous (it is updated in place)")
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    weight = weight.contiguous()
    xr, xs = _row_view(x[:, :, 0])
    out = torch.empty(n, C, 1, dtype=x.dtype, device=x.device)
    _lib.call("gdn_conv_update", _lib.ptr(xr), xs, _lib.ptr(state), _lib.ptr(weight), _lib.ptr(bias),
              _lib.ptr(out), C, n, C, K, _lib.stream_of(x))
    return out


def causal_conv1d_update(hidden_states, conv_state, weight, bias=None, activation=None):
    """HF's decode conv update contract (HF:200-217) on the elem_conv_update kernel.  Several new
    tokens are applied one after another, which gives HF's outputs and final state."""
    if activation not in ("silu", "swish"):
        raise NotImplementedError("causal_conv1d_update: only the SiLU activation is fused")
    T = hidden_states.shape[-1]
    if T == 1:
        return elem_conv_update(hidden_states, conv_state, weight, bias)
    return torch.cat([elem_conv_update(hidden_states[:, :, t:t + 1], conv_state, weight, bias)
                      for t in range(T)], dim=-1)


def gated_rmsnorm(hidden_states, gate, weight, eps=1e-6):
    """silu(gate) * (weight * bf16(x * rsqrt(mean(x^2) + eps))) over the last dim, HF order
    (HF:175-184).  hidden_states, gate [..., D] bf16; weight [D] bf16 or fp32."""
    _lib.require_cuda(hidden_states, gate, weight)
    if hidden_states.dtype != torch.bfloat16 or gate.dtype != torch.bfloat16:
        raise TypeError("gated_rmsnorm: hidden_states and gate must be bfloat16")
    D = hidden_states.shape[-1]
    if gate.shape != hidden_states.shape or weight.shape != (D,):
        raise ValueError("gated_rmsnorm: gate must match hidden_states and weight must be [D]")
    x, xs = _row_view(hidden_states.reshape(-1, D))
    z, zs = _row_view(gate.reshape(-1, D))
    w = weight.contiguous()
    out = torch.empty(hidden_states.shape, dtype=hidden_states.dtype, device=hidden_states.device)
    _lib.call("gdn_gated_rmsnorm", _lib.ptr(x), xs, _lib.ptr(z), zs, _lib.ptr(w), _lib.dtype_code(w),
              _lib.ptr(out), x.shape[0], D, float(eps), _lib.stream_of(x))
    return out


def fused_gated_rmsnorm(self, hidden_states, gate=None):
    """Bound onto Qwen3_5RMSNormGated modules by patch_model (src/cb_engine.py:65-67)."""
    return gated_rmsnorm(hidden_states, gate, self.weight, self.variance_epsilon)


def fused_rmsnorm(self, x):
    """Bound onto bf16 Qwen3_5RMSNorm modules by patch_model (src/cb_engine.py:62-63): HF's
    Qwen3_5RMSNorm.forward -- x * rsqrt(mean(x^2) + eps) in fp32, times (1 + w) in fp32, one bf16
    rounding -- as one gdn_add_rmsnorm launch per call over the rows of x [..., H] bf16 (a
    non-contiguous x, such as q_norm's half of the fused q|gate projection, is copied first)."""
    H = x.shape[-1]
    x2 = x.reshape(-1, H)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    _, y = add_rms_norm(x2, None, self.weight, self.eps)
    return y.view(x.shape)


def gdn_decode_core(mixed, z, a, b, conv_state, conv_weight, A_log, dt_bias, norm_weight, rec_state,
                    num_k_heads, num_v_heads, head_dim, eps=1e-6, conv_bias=None, out=None, active=None):
    """One fused kernel for the GDN decode layer between in_proj_* and out_proj
    (src/cb_engine.py:325-351 with ELEM_CONV): conv update + SiLU, split, gating, l2norm, recurrent
    step, gated RMSNorm.  mixed [N, C] bf16 (pre-conv), z [N, H_v*d] bf16, a, b [N, H_v] bf16;
    conv_state [N, C, K] bf16 and rec_state [N, H_v, d, d] fp32 are updated in place.
    A_log, dt_bias, norm_weight: the layer's parameters (any float dtype; A_log / dt_bias are read in
    fp32 exactly as the reference's ``.float()``).  ``active`` (bool / uint8 [N] on the device, or
    None = all): slots that advance; the others keep their conv and recurrent state and get zero
    output rows -- the held slots of src/cb_tp.py:274-285 without the save / restore copies.
    Returns the normed core [N, H_v*d] bf16."""
    _lib.require_cuda(mixed, z, a, b, conv_state, conv_weight, rec_state)
    # (the per-call host work is kept to what the arguments need: this runs once per layer and step)
    N, C = mixed.shape
    Hk, Hv, D = num_k_heads, num_v_heads, head_dim
    K = conv_weight.shape[-1]
    if C != (2 * Hk + Hv) * D:
        raise ValueError(f"gdn_decode_core: C={C} != (2*{Hk}+{Hv})*{D}")
    if conv_state.shape != (N, C, K) or not conv_state.is_contiguous():
        raise ValueError("gdn_decode_core: conv_state must be a contiguous [N, C, K] tensor")
    if rec_state.shape != (N, Hv, D, D) or rec_state.dtype != torch.float32 or not rec_state.is_contiguous():
        raise ValueError("gdn_decode_core: rec_state must be a contiguous fp32 [N, H_v, d, d] tensor")
    bf16 = torch.bfloat16
    if mixed.dtype != bf16 or z.dtype != bf16 or a.dtype != bf16 or b.dtype != bf16 or conv_state.dtype != bf16 \
            or conv_weight.dtype != bf16:
        for name, t in (("mixed", mixed), ("z", z), ("a", a), ("b", b), ("conv_state", conv_state),
                        ("conv_weight", conv_weight)):
            if t.dtype != bf16:
                raise TypeError(f"gdn_decode_core: {name} must be bfloat16")
    mixed, ms = _row_view(mixed)
    if z.dim() != 2:
        z = z.reshape(N, Hv * D)
    z, zs = _row_view(z)
    if zs % 4 or z.data_ptr() % 8:          # the kernel reads 4 gate values per 8-byte load
        z, zs = z.contiguous(), Hv * D
    if a.dim() != 2:
        a = a.reshape(N, Hv)
    if b.dim() != 2:
        b = b.reshape(N, Hv)
    if a.stride() != b.stride() or a.stride(-1) != 1:
        a, b = a.contiguous(), b.contiguous()
    if not conv_weight.is_contiguous():      # [C, K] or [C, 1, K]: the same memory when contiguous
        conv_weight = conv_weight.contiguous()
    if conv_weight.numel() != C * K:
        raise ValueError(f"gdn_decode_core: conv_weight must hold [C={C}, K={K}]")
    if conv_bias is not None:
        conv_bias = conv_bias.to(bf16).contiguous()
    A32 = A_log if A_log.dtype == torch.float32 and A_log.is_contiguous() else A_log.to(torch.float32).contiguous()
    dt32 = dt_bias if dt_bias.dtype == torch.float32 and dt_bias.is_contiguous() \
        else dt_bias.to(torch.float32).contiguous()
    nw = norm_weight if norm_weight.dtype in (torch.float32, bf16) else norm_weight.float()
    if not nw.is_contiguous() or nw.data_ptr() % 16:
        nw = nw.contiguous().clone()
    if out is None:
        out = torch.empty(N, Hv * D, dtype=bf16, device=mixed.device)
    elif not out.is_contiguous() or out.data_ptr() % 8:
        raise ValueError("gdn_decode_core: out must be a contiguous, 8-byte aligned bf16 [N, H_v*d] tensor")
    if active is not None:
        _lib.require_cuda(active)
        if active.numel() != N:
            raise ValueError(f"gdn_decode_core: active must have N={N} entries")
        active = active.reshape(N).to(torch.uint8).contiguous()
    _lib.call("gdn_decode_fused_masked", mixed.data_ptr(), ms, z.data_ptr(), zs, a.data_ptr(), b.data_ptr(),
              a.stride(0), conv_state.data_ptr(), conv_weight.data_ptr(),
              None if conv_bias is None else conv_bias.data_ptr(), A32.data_ptr(), dt32.data_ptr(), nw.data_ptr(),
              _lib.dtype_code(nw), float(eps), rec_state.data_ptr(), out.data_ptr(),
              None if active is None else active.data_ptr(), N, Hk, Hv, D, K, _lib.stream_of(mixed))
    return out


def patch_model(model, fast_gdn=False, gdn_v2=False):
    """Install the HIP hot-path functions on a transformers Qwen3.5 model (src/cb_engine.py:54-77):
    every Qwen3_5GatedDeltaNet gets ``recurrent_gated_delta_rule`` and, with ``fast_gdn``,
    ``chunk_gated_delta_rule`` (v2 with ``gdn_v2``; v2 is only installed together with fast_gdn,
    as in the reference); every Qwen3_5RMSNormGated gets the fused gated norm and every bf16
    Qwen3_5RMSNorm the fused norm (HF's numerics; the reference's npu_rms_norm rounds 1 + w to the
    input dtype first, a closed rounding not followed here; norms of other dtypes are left to
    transformers).  transformers >= 5.6 calls the module-level functions from
    GatedDeltaNet.forward, so those names are rebound in the modeling module as well."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as M
    from .gdn_chunk_fast import fast_chunk_gated_delta_rule as v1
    from .gdn_chunk_fast2 import fast_chunk_gated_delta_rule_v2 as v2
    chunk_fn = (v2 if gdn_v2 else v1) if fast_gdn else None
    for m in model.modules():
        if isinstance(m, M.Qwen3_5RMSNormGated):
            m.forward = fused_gated_rmsnorm.__get__(m, M.Qwen3_5RMSNormGated)
        elif isinstance(m, M.Qwen3_5RMSNorm) and m.weight.dtype == torch.bfloat16:
            m.forward = fused_rmsnorm.__get__(m, M.Qwen3_5RMSNorm)
        elif isinstance(m, M.Qwen3_5GatedDeltaNet):
            m.recurrent_gated_delta_rule = recurrent_single_step
            if chunk_fn is not None:
                m.chunk_gated_delta_rule = chunk_fn
    M.torch_recurrent_gated_delta_rule = recurrent_single_step
    if chunk_fn is not None:
        M.torch_chunk_gated_delta_rule = chunk_fn
    M.causal_conv1d_update = causal_conv1d_update
    return model


class PackedWeight:
    """A linear weight [N, K] bf16 (nn.Linear layout) repacked once into the decode projection
    kernel's fragment-major layout (every load of the kernel then reads 1 KB contiguous)."""

    def __init__(self, weight):
        _lib.require_cuda(weight)
        N, K = weight.shape
        if weight.dtype != torch.bfloat16 or K % 128:
            raise ValueError("PackedWeight: bf16 [N, K] with K a multiple of 128")
        w = weight.contiguous()
        self.N, self.K = N, K
        self.data = torch.empty(int(_lib.lib().gdn_decode_linear_packed_elems(N, K)), dtype=torch.bfloat16,
                                device=weight.device)
        _lib.call("gdn_decode_linear_pack", _lib.ptr(w), w.stride(0), _lib.ptr(self.data), N, K,
                  _lib.stream_of(w))


def decode_linear(x, weight):
    """x [M, K] bf16 @ weight[N, K]^T (nn.Linear layout, or a PackedWeight) -> [M, N] bf16 for a
    decode step's M <= 16 rows (one token per slot): the GDN layer's in_proj_* / out_proj
    (src/cb_engine.py:320-323, :352) on the weight-streaming projection kernel.  Plain weights of
    shapes it does not take (more rows, K not a multiple of 128, rows not 16-byte aligned) run on
    torch's GEMM."""
    if isinstance(weight, PackedWeight):
        _lib.require_cuda(x)
        M, K = x.shape
        if K != weight.K or M > 16 or x.dtype != torch.bfloat16:
            raise ValueError(f"decode_linear: x {tuple(x.shape)} {x.dtype} does not fit the packed weight "
                             f"[{weight.N}, {weight.K}] (at most 16 bf16 rows)")
        x, xs = _lib.dense_rows(x)
        out = torch.empty(M, weight.N, dtype=torch.bfloat16, device=x.device)
        wb = int(_lib.lib().gdn_decode_linear_workspace_bytes(M, weight.N, K))
        ws = torch.empty(max(wb // 4, 1), dtype=torch.float32, device=x.device) if wb else None
        _lib.call("gdn_decode_linear_packed", _lib.ptr(x), xs, _lib.ptr(weight.data), _lib.ptr(out),
                  out.stride(0), M, weight.N, K, _lib.ptr(ws), wb, _lib.stream_of(x))
        return out
    _lib.require_cuda(x, weight)
    M, K = x.shape
    N = weight.shape[0]
    if (M > 16 or K % 128 or weight.shape[1] != K or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16
            or x.stride(1) != 1 or weight.stride(1) != 1 or x.stride(0) % 8 or weight.stride(0) % 8
            or x.data_ptr() % 16 or weight.data_ptr() % 16):
        return x @ weight.t()
    out = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    wb = int(_lib.lib().gdn_decode_linear_workspace_bytes(M, N, K))
    ws = torch.empty(max(wb // 4, 1), dtype=torch.float32, device=x.device) if wb else None
    _lib.call("gdn_decode_linear", _lib.ptr(x), x.stride(0), _lib.ptr(weight), weight.stride(0), _lib.ptr(out),
              out.stride(0), M, N, K, _lib.ptr(ws), wb, _lib.stream_of(x))
    return out


class Partials:
    """The fp32 split-K partial sums [splits, M, N] of a decode projection (decode_linear_partial):
    the projection's bf16 output is bf16(data.sum(0)) summed in split order, which the consumer
    (add_rms_norm, swiglu) forms itself."""

    def __init__(self, data, splits, M, N):
        self.data, self.splits, self.M, self.N = data, splits, M, N

    def to_bf16(self):
        out = self.data[0].clone()
        for s in range(1, self.splits):
            out += self.data[s]
        return out.to(torch.bfloat16)


def decode_linear_partial(x, weight):
    """decode_linear on a PackedWeight, returning its split-K partial sums (Partials) instead of the
    reduced bf16 output: for a consumer that reduces them itself."""
    _lib.require_cuda(x)
    M, K = x.shape
    if not isinstance(weight, PackedWeight) or K != weight.K or M > 16 or x.dtype != torch.bfloat16:
        raise ValueError("decode_linear_partial: bf16 x [M <= 16, K] and a PackedWeight [N, K]")
    x, xs = _lib.dense_rows(x)
    splits = int(_lib.lib().gdn_decode_linear_splits(M, weight.N, K))
    part = torch.empty(splits, M, weight.N, dtype=torch.float32, device=x.device)
    _lib.call("gdn_decode_linear_packed_partial", _lib.ptr(x), xs, _lib.ptr(weight.data), _lib.ptr(part),
              M, weight.N, K, part.numel() * 4, _lib.stream_of(x))
    return Partials(part, splits, M, weight.N)


def swiglu(gate_up):
    """HF Qwen3_5MLP's act_fn(gate) * up with gate | up as one projection [M, 2m]: a bf16 tensor, or the
    Partials of the gate_up projection (reduced here, no separate reduction)."""
    if isinstance(gate_up, Partials):
        M, m = gate_up.M, gate_up.N // 2
        out = torch.empty(M, m, dtype=torch.bfloat16, device=gate_up.data.device)
        _lib.call("gdn_swiglu_partial", _lib.ptr(gate_up.data), gate_up.splits, _lib.ptr(out), M, m,
                  _lib.stream_of(out))
        return out
    m = gate_up.shape[-1] // 2
    return torch.nn.functional.silu(gate_up[:, :m]) * gate_up[:, m:]


def attn_decode_workspace(n_slots, n_heads, head_dim, cache_len, device):
    """The fp32 workspace gqa_decode_attention needs for these sizes (allocate once, reuse per layer)."""
    nbytes = int(_lib.lib().gdn_attn_decode_workspace_bytes(n_slots, n_heads, head_dim, cache_len))
    if nbytes < 0:
        raise ValueError("attn_decode_workspace: bad sizes")
    return torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=device)


def gqa_decode_attention(proj, pos, q_norm, k_norm, inv_freq, k_cache_t, v_cache, n_heads, kv_heads, head_dim,
                         rotary_dim, eps=1e-6, work=None):
    """HF Qwen3_5Attention.forward at decode (modeling_qwen3_5.py:629-700) after its one fused q|gate|k|v
    projection: q/k Qwen3_5RMSNorm, partial rotary at each slot's position, K and V written into the
    per-slot cache (K transposed [N, kv, hd, T], V [N, kv, T, hd]) at ``pos``, softmax attention over
    positions 0..pos, times sigmoid(gate).  proj [N, (2 nh + 2 kv) hd] bf16 (per head q then gate, then
    k, then v), or that projection's Partials (decode_linear_partial: reduced here, no reduction
    launch), pos [N] int64 on the device.  Returns the gated output [N, nh * hd] bf16 (o_proj's
    input).  Three HIP launches, capturable in a graph."""
    nh, kv, hd = n_heads, kv_heads, head_dim
    part = proj if isinstance(proj, Partials) else None
    if part is not None:
        if part.N != (2 * nh + 2 * kv) * hd:
            raise ValueError("gqa_decode_attention: partials of a [(2 nh + 2 kv) hd]-wide projection expected")
        proj = part.data[0]                      # device, dtype and row count for the checks below
    _lib.require_cuda(proj, pos, q_norm, k_norm, k_cache_t, v_cache)
    N = proj.shape[0]
    T = k_cache_t.shape[-1]
    if ((proj.dtype != torch.bfloat16 and part is None) or proj.stride(1) != 1 or pos.dtype != torch.int64
            or pos.numel() != N
            or tuple(k_cache_t.shape) != (N, kv, hd, T) or tuple(v_cache.shape) != (N, kv, T, hd)
            or not (k_cache_t.is_contiguous() and v_cache.is_contiguous())
            or k_cache_t.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16):
        raise ValueError("gqa_decode_attention: bf16 proj [N, (2 nh + 2 kv) hd], int64 pos [N], contiguous bf16 "
                         "caches K^T [N, kv, hd, T] and V [N, kv, T, hd]")
    qn = q_norm.to(torch.bfloat16).contiguous()
    kn = k_norm.to(torch.bfloat16).contiguous()
    inv = inv_freq.to(torch.float32).contiguous() if rotary_dim else None
    if work is None:
        work = attn_decode_workspace(N, nh, hd, T, proj.device)
    out = torch.empty(N, nh * hd, dtype=torch.bfloat16, device=proj.device)
    rest = (_lib.ptr(pos.contiguous()), _lib.ptr(qn), _lib.ptr(kn), _lib.ptr(inv), _lib.ptr(k_cache_t),
            _lib.ptr(v_cache), _lib.ptr(out), out.stride(0), _lib.ptr(work), work.numel() * 4, N, nh, kv, hd,
            rotary_dim, T, float(eps), _lib.stream_of(proj))
    if part is not None:
        _lib.call("gdn_attn_decode_partial", _lib.ptr(part.data), part.splits, *rest)
    else:
        _lib.call("gdn_attn_decode", _lib.ptr(proj), proj.stride(0), *rest)
    return out


def add_rms_norm(h, delta, weight, eps=1e-6):
    """Residual add + Qwen3_5RMSNorm between decode-step layers (HF modeling_qwen3_5.py):
    h, delta [M, H] bf16 (delta None: norm only; or the Partials of the projection that produced it),
    weight [H] bf16.  Returns (h + delta, norm of it); one kernel instead of the add and the norm's
    chain of elementwise ops."""
    _lib.require_cuda(h, weight)
    M, H = h.shape
    if isinstance(delta, Partials):
        if (delta.M, delta.N) != (M, H) or h.dtype != torch.bfloat16 or not h.is_contiguous():
            raise ValueError(f"add_rms_norm: h must be a contiguous bf16 [{M}, {H}] tensor matching the partials")
        w = weight.to(torch.bfloat16).contiguous()
        x = torch.empty_like(h)
        h_out = torch.empty_like(h)
        _lib.call("gdn_add_rmsnorm_partial", _lib.ptr(h), _lib.ptr(delta.data), delta.splits, _lib.ptr(w),
                  _lib.ptr(h_out), _lib.ptr(x), M, H, float(eps), _lib.stream_of(h))
        return h_out, x
    _lib.require_cuda(delta)
    for name, t in (("h", h), ("delta", delta)):
        if t is not None and (t.dtype != torch.bfloat16 or t.shape != (M, H) or not t.is_contiguous()):
            raise ValueError(f"add_rms_norm: {name} must be a contiguous bf16 [{M}, {H}] tensor")
    w = weight.to(torch.bfloat16).contiguous()
    x = torch.empty_like(h)
    h_out = torch.empty_like(h) if delta is not None else h
    _lib.call("gdn_add_rmsnorm", _lib.ptr(h), _lib.ptr(delta), _lib.ptr(w), _lib.ptr(h_out), _lib.ptr(x), M, H,
              float(eps), _lib.stream_of(h))
    return h_out, x


class GDNSlots:
    """Per-slot GDN state of every GDN layer, laid out as CBEngine keeps it
    (src/cb_engine.py:108-112): conv[i] [N, C, K] bf16, rec[i] [N, H_v, d_k, d_v] fp32."""

    def __init__(self, n_slots, layer_ids, conv_dim, conv_kernel, num_v_heads, head_dim, device):
        self.N = n_slots
        self.conv = {i: torch.zeros(n_slots, conv_dim, conv_kernel, dtype=torch.bfloat16, device=device)
                     for i in layer_ids}
        self.rec = {i: torch.zeros(n_slots, num_v_heads, head_dim, head_dim, dtype=torch.float32,
                                   device=device) for i in layer_ids}

    def reset(self):
        for i in self.conv:
            self.conv[i].zero_()
            self.rec[i].zero_()


def gdn_decode_layer(gd, h, conv_state, rec_state):
    """CBEngine._gdn (src/cb_engine.py:318-352) for one token per slot: projections (torch GEMMs),
    the fused HIP core, out_proj.  ``gd`` carries Qwen3_5GatedDeltaNet's attributes
    (in_proj_qkv, in_proj_z, in_proj_b, in_proj_a, conv1d, A_log, dt_bias, norm, out_proj,
    num_k_heads, num_v_heads, head_k_dim).  h [N, 1, hidden] bf16 -> [N, 1, hidden]."""
    n = h.shape[0]
    mixed = gd.in_proj_qkv(h).reshape(n, -1)
    z = gd.in_proj_z(h).reshape(n, -1)
    b = gd.in_proj_b(h).reshape(n, -1)
    a = gd.in_proj_a(h).reshape(n, -1)
    w = gd.conv1d.weight
    core = gdn_decode_core(mixed, z, a, b, conv_state, w.reshape(w.shape[0], w.shape[-1]), gd.A_log,
                           gd.dt_bias, gd.norm.weight, rec_state, gd.num_k_heads, gd.num_v_heads,
                           gd.head_k_dim, gd.norm.variance_epsilon, gd.conv1d.bias)
    return gd.out_proj(core.reshape(n, 1, -1))


class GDNDecodeGraph:
    """A decode step over several GDN layers captured once as a HIP graph and replayed
    (the GDN part of src/cb_engine.py:123-187).  ``step_fn()`` must read its inputs from static
    buffers; it is run once eagerly (warm-up), then captured."""

    def __init__(self, step_fn, device=None):
        self.step_fn = step_fn
        self.graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(device=device)
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            step_fn()
        torch.cuda.current_stream(device).wait_stream(stream)
        torch.cuda.synchronize(device)
        with torch.cuda.graph(self.graph):
            self.out = step_fn()

    def replay(self):
        self.graph.replay()
        return self.out
