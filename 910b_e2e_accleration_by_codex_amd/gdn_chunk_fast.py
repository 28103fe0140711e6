"""Chunked gated delta rule prefill on the HIP library.

Drop-in for the reference's ``fast_chunk_gated_delta_rule`` (src/gdn_chunk_fast.py:65-142), whose
signature is HF's ``torch_chunk_gated_delta_rule`` (HF modeling_qwen3_5.py:249-260); the v2 name
(src/gdn_chunk_fast2.py:11) runs the same kernel (gdn_chunk_fast2.py).  Semantics kept: q, k are
l2-normalised in their own dtype when ``use_qk_l2norm_in_kernel``, q is scaled by d^-1/2, the
sequence is processed in chunks of 64 with an fp32 running state, the output has query's dtype and
the final state is fp32.  Like the reference it takes any float dtype of q/k/v (fp32, bf16, fp16), head
dims d_k, d_v in {16, 32, 64, 128} and any chunk_size: bf16 q/k/v with d_k = d_v = 128 (the model's
shape) run on the segment-parallel bf16 MFMA kernels, everything else on the generic fp32 kernel
(gdn_chunk_prefill_generic).  Both compute with 64-token chunks: every chunk size gives the same
recurrence in exact arithmetic (the reference's chunk_size only changes its fp32 rounding order).
Added beyond the reference: ``cu_seqlens`` (int32 [n_seq+1]) for packed varlen batches
([1, sum T, H, d] inputs, [n_seq, H_v, d, d] states), the form HF forwards as ``cu_seq_lens_q``.

Also here: the causal conv1d prefill with state capture (src/cb_tp.py:158-164, :236-244, :260),
the gating, and the fused prefill layer core (src/cb_tp.py:153-181, :230-263).
"""
import torch

from . import _lib

CHUNK = 64


def _tokens_view(x, name):
    """[B, T, H, d] -> ([B*T, H, d] tensor with dense (H, d), token stride).  torch gives a size-1
    dimension an arbitrary stride: a single token's stride is never used, a single head's is d."""
    B, T, H, D = x.shape
    ts = x.stride(1) if T > 1 else (x.stride(0) if B > 1 else H * D)
    hs = x.stride(2) if H > 1 else D
    if x.stride(3) != 1 or hs != D or (B > 1 and T > 1 and x.stride(0) != T * ts):
        x, ts = x.clone(memory_format=torch.contiguous_format), H * D
    flat = x.as_strided((B * T, H, D), (ts, D, 1))
    return flat, ts


def _to_device_int32(host, device):
    """int64 host tensor -> int32 device tensor through pinned memory, without waiting for the GPU."""
    if torch.device(device).type == "cpu":
        return host.to(torch.int32)
    staged = torch.empty(host.shape, dtype=torch.int32, pin_memory=True)
    staged.copy_(host)
    return staged.to(device, non_blocking=True)


class Varlen:
    """A packed batch's sequence table, checked once on the host (the kernels index memory with it):
    cu_seqlens 1-D, starting at 0, non-decreasing, ending at the packed token count.  Holds the
    device copies of cu_seqlens and of seq_chunk0 (seq_chunk0[s] = number of 64-token chunks of the
    sequences before s: the workspace slot of the first chunk of sequence s).
    cu_seqlens given on the host (a CPU tensor or a list, as a scheduler holds it) costs no GPU
    wait: the tables go up through pinned memory on the stream.  A device tensor is read back once.
    Build one per batch step and hand it to every op of every layer of that step: the table is the
    same for all of them."""

    def __init__(self, cu_seqlens, T, device):
        if isinstance(cu_seqlens, Varlen):
            raise TypeError("already a Varlen")
        if isinstance(cu_seqlens, (list, tuple)):
            cu = [int(x) for x in cu_seqlens]
        else:
            cu = torch.as_tensor(cu_seqlens).detach().to("cpu", torch.int64).reshape(-1).tolist()
        if len(cu) < 2 or cu[0] != 0 or cu[-1] != T or any(y < x for x, y in zip(cu, cu[1:])):
            raise ValueError(f"cu_seqlens must be non-decreasing from 0 to {T}, got {cu[:8]}...")
        self.T = T
        self.nseq = len(cu) - 1
        s0 = [0]
        for x, y in zip(cu, cu[1:]):
            s0.append(s0[-1] + (y - x + CHUNK - 1) // CHUNK)
        self.total_chunks = s0[-1]
        self.max_len = max(y - x for x, y in zip(cu, cu[1:])) if self.nseq else 0  # the kernels' seq_len bound
        # both tables go up in one pinned copy (the host overhead of a layer call with a fresh table)
        both = _to_device_int32(torch.tensor(cu + s0, dtype=torch.int64), device)
        self.cu, self.seq_chunk0 = both[:len(cu)], both[len(cu):]


def _varlen(cu_seqlens, B, T, device):
    if B != 1:
        raise ValueError("cu_seqlens needs packed inputs with batch size 1")
    if isinstance(cu_seqlens, Varlen):
        if cu_seqlens.T != T:
            raise ValueError(f"Varlen built for {cu_seqlens.T} tokens, inputs hold {T}")
        return cu_seqlens
    return Varlen(cu_seqlens, T, device)


def _seq_args(B, T, cu_seqlens, device):
    """(device int32 cu_seqlens | None, n_seq, per-sequence length for the uniform case)."""
    if cu_seqlens is None:
        return None, B, T
    vl = _varlen(cu_seqlens, B, T, device)
    return vl.cu, vl.nseq, 0


def _chunk_table(B, T, cu_seqlens, device):
    """(device cu_seqlens | None, device seq_chunk0 | None, n_seq, seq_len, total_chunks)."""
    if cu_seqlens is None:
        return None, None, B, T, B * ((T + CHUNK - 1) // CHUNK)
    vl = _varlen(cu_seqlens, B, T, device)
    return vl.cu, vl.seq_chunk0, vl.nseq, vl.max_len, vl.total_chunks


class Rows:
    """Slot rows of a batch's sequences (int [n_seq]), checked once on the host: every row in
    [0, n_rows).  Host input (CPU tensor / list) costs no GPU wait; a device tensor is read back once."""

    def __init__(self, state_rows, nseq, n_rows, device):
        if isinstance(state_rows, (list, tuple)):
            rows = [int(x) for x in state_rows]
        else:
            rows = torch.as_tensor(state_rows).detach().to("cpu", torch.int64).reshape(-1).tolist()
        if len(rows) != nseq:
            raise ValueError(f"state_rows must hold one row per sequence ({nseq})")
        if nseq and (min(rows) < 0 or max(rows) >= n_rows):
            raise ValueError(f"state_rows must lie in [0, {n_rows})")
        self.nseq, self.n_rows = nseq, n_rows
        self.dev = _to_device_int32(torch.tensor(rows, dtype=torch.int64), device)


def _check_rows(state_rows, nseq, n_rows, device):
    """Device int32 slot rows, checked (see Rows)."""
    if isinstance(state_rows, Rows):
        if state_rows.nseq != nseq or state_rows.n_rows != n_rows:
            raise ValueError(f"Rows built for {state_rows.nseq} sequences / {state_rows.n_rows} rows, "
                             f"call has {nseq} / {n_rows}")
        return state_rows.dev
    return Rows(state_rows, nseq, n_rows, device).dev


FAST = "bfloat16 query/key/value with head dims 128"
DIMS = (16, 32, 64, 128)
FLOATS = (torch.float32, torch.bfloat16, torch.float16)


def check_chunk_args(query, key, value, chunk_size):
    """The reference's argument domain (src/gdn_chunk_fast2.py:11-29): q/k/v of one float dtype
    (fp32, bf16 or fp16), d_k = q/k's last dim and d_v = v's in {16, 32, 64, 128}, chunk_size a
    positive integer (computed with 64-token chunks: the same recurrence).  Returns True when the
    call takes the segment-parallel bf16 kernels (bf16, d_k = d_v = 128), False for the generic
    fp32 kernel; anything outside the domain raises ValueError before any GPU work."""
    if not isinstance(chunk_size, int) or isinstance(chunk_size, bool) or chunk_size < 1:
        raise ValueError(f"chunk_gated_delta_rule: chunk_size must be a positive integer, got {chunk_size!r}")
    if not (query.dtype == key.dtype == value.dtype) or query.dtype not in FLOATS:
        raise ValueError(f"chunk_gated_delta_rule: query/key/value dtypes {query.dtype}/{key.dtype}/{value.dtype} "
                         f"are not supported (one of float32, bfloat16, float16 for all three)")
    if query.dim() != 4 or query.shape[-1] not in DIMS or value.shape[-1] not in DIMS:
        raise ValueError(f"chunk_gated_delta_rule: head dims {query.shape[-1]} / {value.shape[-1]} are not supported "
                         f"(d_k, d_v in {DIMS})")
    return query.dtype == torch.bfloat16 and query.shape[-1] == 128 and value.shape[-1] == 128


def chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None,
                           output_final_state=False, use_qk_l2norm_in_kernel=False, cu_seqlens=None,
                           state_rows=None, final_state_out=None, norm_gate=None, **kwargs):
    """query/key [B,T,Hqk,d] (Hqk = Hv after repeat_interleave, or Hv/r key heads read by value
    head h as h // r), value [B,T,Hv,d] bf16, g [B,T,Hv] (log decay, read in fp32), beta
    [B,T,Hv], initial_state [B or n_seq, Hv, d, d] | None.
    Returns (out [B,T,Hv,d] query.dtype, final_state [B or n_seq,Hv,d,d] fp32 | None).
    Slot rows (added for a continuous-batching engine): with ``state_rows`` (int [n_seq]) the states
    live in slot buffers -- ``initial_state`` (or None = zero) and ``final_state_out`` are fp32
    [n_rows, Hv, d, d], sequence s uses row state_rows[s], and the two may be the same tensor; the
    final state is then written there and returned.
    Fused output norm (the GDN layer's Qwen3_5RMSNormGated, src/cb_tp.py:171-176): with
    ``norm_gate`` = (z, norm_weight, eps), z bf16 [B*T, >= Hv*d] rows with unit inner stride (head h
    of token t at z[t, h*d:(h+1)*d]) and norm_weight [d] bf16 or fp32, the returned rows are
    gated_rmsnorm(out, z, norm_weight, eps) -- computed by the output kernel before the store."""
    fast = check_chunk_args(query, key, value, chunk_size)
    _lib.require_cuda(query, key, value, g, beta, initial_state)
    B, T, Hqk, D = query.shape
    Hv, Dv = value.shape[2], value.shape[3]
    if key.shape != query.shape or tuple(value.shape[:2]) != (B, T):
        raise ValueError(f"chunk_gated_delta_rule: shape mismatch q{tuple(query.shape)} "
                         f"k{tuple(key.shape)} v{tuple(value.shape)}")
    if Hv % Hqk:
        raise ValueError(f"chunk_gated_delta_rule: value heads {Hv} not a multiple of query/key heads {Hqk}")
    if tuple(g.shape) != (B, T, Hv) or tuple(beta.shape) != (B, T, Hv):
        raise ValueError("chunk_gated_delta_rule: g and beta must be [B, T, Hv]")
    if norm_gate is not None and not fast:
        raise ValueError(f"chunk_gated_delta_rule: the fused output norm needs {FAST}")
    dev = query.device
    if fast:
        cu, seq_chunk0, nseq, seq_len, total_chunks = _chunk_table(B, T, cu_seqlens, dev)
    else:  # the generic kernel walks each sequence itself: no chunk table
        cu, nseq, seq_len = _seq_args(B, T, cu_seqlens, dev)
        seq_chunk0, total_chunks = None, 0
    q, qs = _tokens_view(query, "query")
    k, ks = _tokens_view(key, "key")
    v, vs = _tokens_view(value, "value")
    g32 = g.to(torch.float32).contiguous()
    if beta.dtype not in ((torch.float32, torch.bfloat16) if fast else FLOATS):
        beta = beta.to(torch.float32)
    beta = beta.contiguous()
    rows, n_rows = None, nseq
    if state_rows is not None:
        if final_state_out is None:
            raise ValueError("chunk_gated_delta_rule: state_rows needs final_state_out (the slot buffer)")
        n_rows = final_state_out.shape[0]
        for name, t in (("final_state_out", final_state_out), ("initial_state", initial_state)):
            if t is not None and (tuple(t.shape) != (n_rows, Hv, D, Dv) or t.dtype != torch.float32
                                  or not t.is_contiguous() or t.device != dev):
                raise ValueError(f"chunk_gated_delta_rule: {name} must be a contiguous fp32 "
                                 f"[{n_rows},{Hv},{D},{Dv}] slot buffer on {dev}")
        rows = _check_rows(state_rows, nseq, n_rows, dev)
        init, final = initial_state, final_state_out
    else:
        init = None
        if initial_state is not None:
            if tuple(initial_state.shape) != (nseq, Hv, D, Dv):
                raise ValueError(f"chunk_gated_delta_rule: initial_state must be [{nseq},{Hv},{D},{Dv}]")
            init = initial_state.to(torch.float32).contiguous()
        final = torch.empty(nseq, Hv, D, Dv, dtype=torch.float32, device=dev) if output_final_state else None
    out = torch.empty(B, T, Hv, Dv, dtype=query.dtype, device=dev)
    if not fast:
        _lib.call("gdn_chunk_prefill_generic", _lib.ptr(q), qs, _lib.ptr(k), ks, _lib.ptr(v), vs, _lib.ptr(g32),
                  _lib.ptr(beta), _lib.dtype_code(beta), _lib.ptr(init), _lib.ptr(final), _lib.ptr(rows), n_rows,
                  _lib.ptr(out), B * T, _lib.ptr(cu), nseq, seq_len, Hqk, Hv, D, Dv, _lib.dtype_code(query),
                  int(bool(use_qk_l2norm_in_kernel)), _lib.stream_of(query))
        return out, final
    wbytes = int(_lib.lib().gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv))
    work = torch.empty(max(wbytes, 1), dtype=torch.uint8, device=dev)
    args = (_lib.ptr(q), qs, _lib.ptr(k), ks, _lib.ptr(v), vs, _lib.ptr(g32), _lib.ptr(beta),
            _lib.dtype_code(beta), _lib.ptr(init), _lib.ptr(final), _lib.ptr(rows), n_rows, _lib.ptr(out), B * T,
            _lib.ptr(cu), _lib.ptr(seq_chunk0), total_chunks, nseq, seq_len, Hqk, Hv, D, _lib.dtype_code(query),
            int(bool(use_qk_l2norm_in_kernel)))
    if norm_gate is None:
        _lib.call("gdn_chunk_prefill_rows", *args, _lib.ptr(work), wbytes, _lib.stream_of(query))
        return out, final
    z, norm_weight, eps = norm_gate
    _lib.require_cuda(z, norm_weight)
    z = z.reshape(B * T, -1)
    if z.dtype != torch.bfloat16 or z.shape[1] < Hv * D or z.device != dev:
        raise ValueError(f"chunk_gated_delta_rule: norm gate must be bf16 [{B * T}, >= {Hv * D}] on {dev}")
    z, zs = _lib.dense_rows(z)
    if tuple(norm_weight.shape) != (D,) or norm_weight.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"chunk_gated_delta_rule: norm weight must be bf16 or fp32 [{D}]")
    w = norm_weight.contiguous()
    _lib.call("gdn_chunk_prefill_rows_gated", *args, _lib.ptr(z), zs, _lib.ptr(w), _lib.dtype_code(w),
              float(eps), _lib.ptr(work), wbytes, _lib.stream_of(query))
    return out, final


def fast_chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None,
                                output_final_state=False, use_qk_l2norm_in_kernel=False, **kwargs):
    """The v1 name (src/gdn_chunk_fast.py:65-75); same kernel as v2."""
    return chunk_gated_delta_rule(query, key, value, g, beta, chunk_size, initial_state,
                                  output_final_state, use_qk_l2norm_in_kernel, **kwargs)


def _unit_lower_inv(X, base=16):
    """(I - X)^-1 for strictly lower X [..., 64, 64] fp32 on the GPU, by the routine the chunked
    prefill's inverse kernel runs (reg_inv64: 16x16 diagonal blocks by forward substitution, the
    blocks below them on the fp32 MFMA, in registers), the blocking of src/gdn_chunk_fast.py:33-62."""
    _lib.require_cuda(X)
    if X.shape[-1] != 64 or X.shape[-2] != 64:
        raise ValueError("_unit_lower_inv: the kernel inverts 64x64 blocks")
    Xf = X.to(torch.float32).contiguous()
    out = torch.empty_like(Xf)
    batch = Xf.numel() // (64 * 64)
    _lib.call("gdn_unit_lower_inv", _lib.ptr(Xf), _lib.ptr(out), batch, 64, _lib.stream_of(Xf))
    return out


def chunk_inverse_records(key, g, beta, use_qk_l2norm_in_kernel=True, cu_seqlens=None, num_v_heads=None):
    """What the chunked prefill's first kernel hands to its output pass, dense (for checking it on
    its own): returns (T [n_chunks, Hv, 64, 64] fp32, factors [n_chunks, Hv, 64] fp32 | None).
    T[c, h, i, j] = (I - X)^-1[i, j] beta_j of chunk c, head h (X = -(beta_i k_i.k_j
    e^{G_i - G_j})_{i>j}), the bf16 values the kernel stores; factors = the K rows' l2norm factors
    bf16(rsqrt(sum k^2 + 1e-6)).  Chunks are numbered sequence by sequence.  key [B, T, Hk, 128]
    bf16, g [B, T, Hv] (fp32), beta [B, T, Hv] (bf16 or fp32).  src/gdn_chunk_fast2.py:31-43."""
    _lib.require_cuda(key, g, beta)
    B, T, Hk, D = key.shape
    Hv = g.shape[-1] if num_v_heads is None else num_v_heads
    if key.dtype != torch.bfloat16 or D != 128:
        raise ValueError("chunk_inverse_records: key must be bf16 with head dim 128")
    if tuple(g.shape) != (B, T, Hv) or tuple(beta.shape) != (B, T, Hv) or Hv % Hk:
        raise ValueError("chunk_inverse_records: g, beta must be [B, T, Hv] with Hv a multiple of Hk")
    dev = key.device
    cu, seq_chunk0, nseq, seq_len, total_chunks = _chunk_table(B, T, cu_seqlens, dev)
    k, ks = _tokens_view(key, "key")
    g32 = g.to(torch.float32).contiguous()
    if beta.dtype not in (torch.float32, torch.bfloat16):
        beta = beta.to(torch.float32)
    beta = beta.contiguous()
    t_out = torch.empty(total_chunks, Hv, 64, 64, dtype=torch.float32, device=dev)
    f_out = torch.empty(total_chunks, Hv, 64, dtype=torch.float32, device=dev) if use_qk_l2norm_in_kernel else None
    wbytes = int(_lib.lib().gdn_chunk_prefill_workspace_bytes(total_chunks, nseq, Hv))
    work = torch.empty(max(wbytes, 1), dtype=torch.uint8, device=dev)
    _lib.call("gdn_chunk_prefill_inverse", _lib.ptr(k), ks, _lib.ptr(g32), _lib.ptr(beta), _lib.dtype_code(beta),
              B * T, _lib.ptr(cu), _lib.ptr(seq_chunk0), total_chunks, nseq, seq_len, Hk, Hv, D, _lib.BF16,
              int(bool(use_qk_l2norm_in_kernel)), _lib.ptr(t_out), _lib.ptr(f_out), _lib.ptr(work), wbytes,
              _lib.stream_of(key))
    return t_out, f_out


def causal_conv1d_prefill(x, weight, bias=None, history=None, cu_seqlens=None, state_rows=None, state_out=None):
    """Depthwise causal conv (kernel K) + SiLU over prompts, plus the decode conv state they leave.
    x [B, C, L] bf16 (HF layout; token-major memory such as ``mixed_qkv.transpose(1, 2)`` is read
    in place); history [n_seq, C, K] | None (None = fresh prompt, zero history: F.conv1d with
    padding K-1, src/cb_tp.py:163-164; given = the previous K inputs, src/cb_tp.py:236-244).
    Returns (out [B, C, L] bf16 with token-major memory, state [n_seq, C, K] = the last K inputs,
    left zero-padded, src/cb_tp.py:158-162, :260).
    Slot rows: with ``state_rows`` (int [n_seq]) ``history`` (or None = zero) and ``state_out`` are
    bf16 [n_rows, C, K] slot buffers, sequence s uses row state_rows[s], and the two may be the same
    tensor; the new states are written there and ``state_out`` is returned."""
    _lib.require_cuda(x, weight, bias, history)
    B, C, L = x.shape
    K = weight.shape[-1]
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("causal_conv1d_prefill: x and weight must be bfloat16")
    xt = x.transpose(1, 2)                                   # [B, L, C]
    xs = xt.stride(1) if L > 1 else (xt.stride(0) if B > 1 else C)  # token row stride (a size-1 dim's
    if (xt.stride(2) != 1 or (B > 1 and L > 1 and xt.stride(0) != L * xs) or xs % 8  # stride is arbitrary)
            or xt.data_ptr() % 16):
        xt, xs = xt.clone(memory_format=torch.contiguous_format), C  # the kernel reads 16-byte row pieces
    cu, nseq, seq_len = _seq_args(B, L, cu_seqlens, x.device)
    w = weight.reshape(C, K).contiguous()
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    rows, n_rows = None, nseq
    if state_rows is not None:
        if state_out is None:
            raise ValueError("causal_conv1d_prefill: state_rows needs state_out (the slot buffer)")
        n_rows = state_out.shape[0]
        for name, t in (("state_out", state_out), ("history", history)):
            if t is not None and (tuple(t.shape) != (n_rows, C, K) or t.dtype != torch.bfloat16
                                  or not t.is_contiguous() or t.device != x.device):
                raise ValueError(f"causal_conv1d_prefill: {name} must be a contiguous bf16 [{n_rows},{C},{K}] "
                                 f"slot buffer on {x.device}")
        rows = _check_rows(state_rows, nseq, n_rows, x.device)
        state = state_out
    else:
        if history is not None:
            if tuple(history.shape) != (nseq, C, K):
                raise ValueError(f"causal_conv1d_prefill: history must be [{nseq},{C},{K}]")
            history = history.to(torch.bfloat16).contiguous()
        state = torch.empty(nseq, C, K, dtype=torch.bfloat16, device=x.device)
    out = torch.empty(B, L, C, dtype=torch.bfloat16, device=x.device)
    _lib.call("gdn_conv_prefill_rows", _lib.ptr(xt), xs, _lib.ptr(w), _lib.ptr(bias),
              _lib.ptr(history), _lib.ptr(out), _lib.ptr(state), _lib.ptr(rows), n_rows, B * L, _lib.ptr(cu),
              nseq, seq_len, C, K, _lib.stream_of(x))
    return out.transpose(1, 2), state


def gdn_gating(a, b, A_log, dt_bias):
    """beta = sigmoid(b) (b's dtype, bf16), g = -exp(A_log) * softplus(a + dt_bias) fp32
    (src/cb_engine.py:337-338).  a, b [..., Hv] bf16."""
    _lib.require_cuda(a, b)
    Hv = a.shape[-1]
    a2 = a.reshape(-1, Hv)
    b2 = b.reshape(-1, Hv)
    if a2.stride() != b2.stride() or a2.stride(-1) != 1:
        a2, b2 = a2.contiguous(), b2.contiguous()
    beta = torch.empty(a2.shape, dtype=torch.bfloat16, device=a.device)
    g = torch.empty(a2.shape, dtype=torch.float32, device=a.device)
    _lib.call("gdn_gating", _lib.ptr(a2), _lib.ptr(b2), a2.stride(0),
              _lib.ptr(A_log.to(torch.float32).contiguous()), _lib.ptr(dt_bias.to(torch.float32).contiguous()),
              _lib.ptr(beta), _lib.ptr(g), a2.shape[0], Hv, _lib.stream_of(a))
    return beta.reshape(b.shape), g.reshape(a.shape)


def gdn_prefill_core(mixed_qkv, z, a, b, conv_weight, A_log, dt_bias, norm_weight, num_k_heads,
                     num_v_heads, head_dim, cu_seqlens=None, conv_history=None, initial_state=None,
                     eps=1e-6, chunk_size=64, conv_bias=None, slots=None, conv_slots=None, rec_slots=None,
                     continuation=False):
    """GDN prefill layer between in_proj_* and out_proj for one or more packed prompts
    (src/cb_tp.py:153-181 fresh, :230-263 continued): conv prefill + SiLU, split q|k|v, gating,
    chunked rule with l2norm (value head h reads key head h // r, no repeat_interleave copy),
    gated RMSNorm (fused into the rule's output kernel) -- one call of gdn_prefill_layer_rows, whose
    first launch does the conv, the conv state, the gating and the segment table.  mixed_qkv [T, C] bf16 (pre-conv),
    z [T, Hv*d], a, b [T, Hv]; cu_seqlens int [n_seq+1] (host or device) | Varlen | None -- host
    lengths, as the scheduler holds them, keep the call free of GPU waits; conv_history [n_seq, C, K] | None;
    initial_state [n_seq, Hv, d, d] | None.
    Returns (core [T, Hv*d] bf16, conv_state [n_seq, C, K] bf16, rec_state [n_seq, Hv, d, d] fp32).
    Slot rows (the engine's state buffers, src/cb_engine.py:198-205, src/cb_tp.py:178-179, :256-262):
    with ``slots`` (int [n_seq]) the states go straight into rows slots[s] of ``conv_slots``
    [N, C, K] bf16 and ``rec_slots`` [N, Hv, d, d] fp32, and with ``continuation`` each sequence
    first reads its conv history and initial state from those rows (a later chunk of a prompt);
    then (core, conv_slots, rec_slots) is returned and conv_history / initial_state are not used."""
    _lib.require_cuda(mixed_qkv, z, a, b, conv_weight, A_log, dt_bias, norm_weight, conv_history, initial_state)
    T, C = mixed_qkv.shape
    Hk, Hv, D = num_k_heads, num_v_heads, head_dim
    if C != (2 * Hk + Hv) * D:
        raise ValueError(f"gdn_prefill_core: C={C} != (2*{Hk}+{Hv})*{D}")
    if not isinstance(chunk_size, int) or chunk_size < 1:
        raise ValueError(f"gdn_prefill_core: chunk_size must be a positive integer, got {chunk_size!r}")
    if D != 128:
        raise ValueError(f"gdn_prefill_core: the fused layer takes head dim 128 (got {D})")
    if mixed_qkv.dtype != torch.bfloat16 or conv_weight.dtype != torch.bfloat16:
        raise TypeError("gdn_prefill_core: mixed_qkv and conv_weight must be bfloat16")
    dev = mixed_qkv.device
    w = conv_weight if conv_weight.is_contiguous() else conv_weight.contiguous()  # [C, K] or [C, 1, K]
    K = w.numel() // C
    if w.numel() != C * K:
        raise ValueError(f"gdn_prefill_core: conv_weight must hold [C={C}, K]")
    if cu_seqlens is not None:  # checked and uploaded once (a Varlen is used as it is)
        vl = _varlen(cu_seqlens, 1, T, dev)
        cu, chunk0, nseq, seq_len, total_chunks = vl.cu, vl.seq_chunk0, vl.nseq, vl.max_len, vl.total_chunks
    else:
        cu, chunk0, nseq, seq_len, total_chunks = None, None, 1, T, (T + CHUNK - 1) // CHUNK
    x, xs = _lib.dense_rows(mixed_qkv)
    z2 = z if z.dim() == 2 else z.reshape(T, -1)
    if z2.dtype != torch.bfloat16 or z2.shape[0] != T or z2.shape[1] < Hv * D:
        raise ValueError(f"gdn_prefill_core: z must be bf16 [{T}, >= {Hv * D}]")
    z2, zs = _lib.dense_rows(z2)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise TypeError(f"gdn_prefill_core: a and b must be bfloat16 (got {a.dtype}, {b.dtype})")
    if a.numel() != T * Hv or b.numel() != T * Hv:
        raise ValueError(f"gdn_prefill_core: a and b must hold [{T}, {Hv}] values")
    if A_log.numel() != Hv or dt_bias.numel() != Hv:
        raise ValueError(f"gdn_prefill_core: A_log and dt_bias must hold {Hv} values "
                         f"(got {A_log.numel()}, {dt_bias.numel()})")
    if conv_bias is not None and conv_bias.numel() != C:
        raise ValueError(f"gdn_prefill_core: conv_bias must hold C={C} values (got {conv_bias.numel()})")
    a2 = a if a.dim() == 2 else a.reshape(T, Hv)
    b2 = b if b.dim() == 2 else b.reshape(T, Hv)
    if T > 1 and (a2.stride() != b2.stride() or a2.stride(-1) != 1):
        a2, b2 = a2.contiguous(), b2.contiguous()
    ab_rs = a2.stride(0) if T > 1 else Hv  # (one row: its stride is never used)
    if T == 1 and (a2.stride(-1) != 1 or b2.stride(-1) != 1):
        a2, b2 = a2.contiguous(), b2.contiguous()
    bias = conv_bias.to(torch.bfloat16).contiguous() if conv_bias is not None else None
    A32 = A_log if A_log.dtype == torch.float32 and A_log.is_contiguous() else A_log.to(torch.float32).contiguous()
    dt32 = dt_bias if dt_bias.dtype == torch.float32 and dt_bias.is_contiguous() \
        else dt_bias.to(torch.float32).contiguous()
    nw = norm_weight if norm_weight.is_contiguous() else norm_weight.contiguous()
    if nw.shape != (D,) or nw.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"gdn_prefill_core: norm weight must be bf16 or fp32 [{D}]")
    if slots is not None:
        if conv_slots is None or rec_slots is None:
            raise ValueError("gdn_prefill_core: slots needs conv_slots and rec_slots")
        n_rows = conv_slots.shape[0]
        if rec_slots.shape[0] != n_rows:
            raise ValueError("gdn_prefill_core: conv_slots and rec_slots must hold the same slot count")
        if (tuple(conv_slots.shape) != (n_rows, C, K) or conv_slots.dtype != torch.bfloat16
                or not conv_slots.is_contiguous() or conv_slots.device != dev):
            raise ValueError(f"gdn_prefill_core: conv_slots must be a contiguous bf16 [{n_rows},{C},{K}] slot buffer")
        if (tuple(rec_slots.shape) != (n_rows, Hv, D, D) or rec_slots.dtype != torch.float32
                or not rec_slots.is_contiguous() or rec_slots.device != dev):
            raise ValueError(f"gdn_prefill_core: rec_slots must be a contiguous fp32 [{n_rows},{Hv},{D},{D}] "
                             "slot buffer")
        rows = _check_rows(slots, nseq, n_rows, dev)
        hist, conv_state = (conv_slots if continuation else None), conv_slots
        init, rec = (rec_slots if continuation else None), rec_slots
    else:
        n_rows, rows = nseq, None
        hist = None
        if conv_history is not None:
            if tuple(conv_history.shape) != (nseq, C, K):
                raise ValueError(f"gdn_prefill_core: conv_history must be [{nseq},{C},{K}]")
            hist = conv_history.to(torch.bfloat16).contiguous()
        conv_state = torch.empty(nseq, C, K, dtype=torch.bfloat16, device=dev)
        init = None
        if initial_state is not None:
            if tuple(initial_state.shape) != (nseq, Hv, D, D):
                raise ValueError(f"gdn_prefill_core: initial_state must be [{nseq},{Hv},{D},{D}]")
            init = initial_state.to(torch.float32).contiguous()
        rec = torch.empty(nseq, Hv, D, D, dtype=torch.float32, device=dev)
    core = torch.empty(T, Hv * D, dtype=torch.bfloat16, device=dev)
    wbytes = int(_lib.lib().gdn_prefill_layer_workspace_bytes(T, total_chunks, nseq, Hk, Hv, D))
    work = torch.empty(max(wbytes, 1), dtype=torch.uint8, device=dev)
    p = _lib.ptr_int
    _lib.call("gdn_prefill_layer_rows", x.data_ptr(), xs, z2.data_ptr(), zs, a2.data_ptr(),
              b2.data_ptr(), ab_rs, w.data_ptr(), p(bias), A32.data_ptr(), dt32.data_ptr(), nw.data_ptr(),
              _lib.dtype_code(nw), float(eps), p(hist), conv_state.data_ptr(), p(init), rec.data_ptr(),
              p(rows), n_rows, core.data_ptr(), T, p(cu), p(chunk0), total_chunks, nseq,
              seq_len, Hk, Hv, D, K, work.data_ptr(), wbytes, _lib.stream_of(mixed_qkv))
    return core, conv_state, rec
