"""Single-token gated delta rule on the HIP library (drop-in for src/recurrent_single_step.py:8-32).

Same signature, dtypes and semantics as the reference: q, k are l2-normalised in their own dtype
when ``use_qk_l2norm_in_kernel``, the update runs in fp32, the output has query's dtype and the
returned state is a NEW fp32 tensor (the input state is not mutated).  ``inplace=True`` is an
opt-in for callers that own the state (the engine): the kernel then updates ``initial_state`` in
place and returns it, so a following ``copy_`` of it onto itself can be skipped.
For T > 1 the reference falls back to the token loop (src/recurrent_single_step.py:10-13); here
the same loop runs one HIP step per token.
"""
import torch

from . import _lib


def _rows(x):
    """[N, H, D] view whose H and D are dense; returns (tensor, row stride)."""
    if x.stride(-1) != 1 or x.stride(-2) != x.shape[-1]:
        x = x.contiguous()
    return x, x.stride(0)


def _step(q, k, v, g, beta, state_in, state_out, out, use_l2):
    """q,k [N,Hqk,D], v [N,Hv,D], g [N,Hv] fp32, beta [N,Hv], out [N,Hv,D] (dense)."""
    N, Hqk, D = q.shape
    Hv = v.shape[1]
    q, qs = _rows(q)
    k, ks = _rows(k)
    v, vs = _rows(v)
    _lib.call("gdn_recurrent_step", _lib.ptr(q), qs, _lib.ptr(k), ks, _lib.ptr(v), vs, _lib.ptr(g),
              _lib.ptr(beta), _lib.dtype_code(beta), _lib.ptr(state_in), _lib.ptr(state_out),
              _lib.ptr(out), N, Hqk, Hv, D, _lib.dtype_code(q), int(bool(use_l2)), _lib.stream_of(q))


def recurrent_single_step(query, key, value, g, beta, initial_state, output_final_state,
                          use_qk_l2norm_in_kernel=False, inplace=False, **kwargs):
    """query/key [N,T,Hqk,D] (Hqk == Hv after repeat_interleave, or Hv/r key heads), value
    [N,T,Hv,D] (bf16 or fp32, same dtype), g [N,T,Hv] (log decay), beta [N,T,Hv],
    initial_state [N,Hv,D,D] or None.  Returns (out [N,T,Hv,D] in query.dtype, state | None)."""
    if kwargs.get("cu_seqlens") is not None:
        raise NotImplementedError("recurrent_single_step: cu_seqlens is not supported (dense slots)")
    _lib.require_cuda(query, key, value, g, beta, initial_state)
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise TypeError("recurrent_single_step: query, key and value must share a dtype")
    N, T, Hqk, D = query.shape
    Hv = value.shape[2]
    if key.shape != query.shape or value.shape[:2] != (N, T) or value.shape[3] != D:
        raise ValueError(f"recurrent_single_step: shape mismatch q{tuple(query.shape)} "
                         f"k{tuple(key.shape)} v{tuple(value.shape)}")
    if tuple(g.shape) != (N, T, Hv) or tuple(beta.shape) != (N, T, Hv):
        raise ValueError("recurrent_single_step: g and beta must be [N, T, Hv]")
    g = g.to(torch.float32)
    if beta.dtype not in (torch.float32, torch.bfloat16):
        beta = beta.to(torch.float32)
    state_in = None
    if initial_state is not None:
        if tuple(initial_state.shape) != (N, Hv, D, D):
            raise ValueError(f"recurrent_single_step: state must be [{N},{Hv},{D},{D}]")
        if inplace and (initial_state.dtype != torch.float32 or not initial_state.is_contiguous()):
            raise ValueError("recurrent_single_step: inplace needs a contiguous fp32 state")
        state_in = initial_state if (initial_state.dtype == torch.float32
                                     and initial_state.is_contiguous()) else \
            initial_state.to(torch.float32).contiguous()
    if inplace and initial_state is not None:
        state_out = state_in
    else:
        state_out = torch.empty(N, Hv, D, D, dtype=torch.float32, device=query.device)
    out = torch.empty(N, T, Hv, D, dtype=query.dtype, device=query.device)
    if T == 1:
        _step(query[:, 0], key[:, 0], value[:, 0], g[:, 0].contiguous(), beta[:, 0].contiguous(),
              state_in, state_out, out[:, 0], use_qk_l2norm_in_kernel)
    else:
        cur = state_in
        step_out = torch.empty(N, Hv, D, dtype=query.dtype, device=query.device)
        for t in range(T):
            _step(query[:, t], key[:, t], value[:, t], g[:, t].contiguous(), beta[:, t].contiguous(),
                  cur, state_out, step_out, use_qk_l2norm_in_kernel)
            out[:, t].copy_(step_out)
            cur = state_out
    return out, (state_out if output_final_state else None)
