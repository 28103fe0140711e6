"""ctypes binding of libgdn_mi355x.so, the C-ABI HIP library (declared in include/gdn_mi355x.h).

torch is imported first so that the HIP runtime torch ships is the one already loaded in the
process; the library then binds to it by soname, and the raw stream handles torch hands out are
valid for it.  There is no CPU fallback: if the library is missing or no GPU is visible every op
raises.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgdn_mi355x.so")

F32, BF16, F16 = 0, 1, 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

_SIGNATURES = {
    "gdn_version": ([], _I),
    "gdn_last_error": ([], ctypes.c_char_p),
    "gdn_limits": ([_P, _P, _P], _I),
    "gdn_recurrent_step": ([_P, _L, _P, _L, _P, _L, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "gdn_conv_update": ([_P, _L, _P, _P, _P, _P, _L, _I, _I, _I, _P], _I),
    "gdn_gated_rmsnorm": ([_P, _L, _P, _L, _P, _I, _P, _L, _I, _F, _P], _I),
    "gdn_decode_fused": ([_P, _L, _P, _L, _P, _P, _L, _P, _P, _P, _P, _P, _P, _I, _F, _P, _P, _I, _I, _I,
                          _I, _I, _P], _I),
    "gdn_unit_lower_inv": ([_P, _P, _L, _I, _P], _I),
    "gdn_chunk_prefill": ([_P, _L, _P, _L, _P, _L, _P, _P, _I, _P, _P, _P, _L, _P, _P, _L, _I, _I, _I, _I,
                           _I, _I, _I, _P, _L, _P], _I),
    "gdn_chunk_prefill_workspace_bytes": ([_L, _I, _I], _L),
    "gdn_prefill_layer_workspace_bytes": ([_L, _L, _I, _I, _I, _I], _L),
    "gdn_decode_linear_workspace_bytes": ([_I, _L, _L], _L),
    "gdn_decode_linear": ([_P, _L, _P, _L, _P, _L, _I, _L, _L, _P, _L, _P], _I),
    "gdn_decode_linear_packed_elems": ([_L, _L], _L),
    "gdn_decode_linear_pack": ([_P, _L, _P, _L, _L, _P], _I),
    "gdn_decode_linear_packed": ([_P, _L, _P, _P, _L, _I, _L, _L, _P, _L, _P], _I),
    "gdn_add_rmsnorm": ([_P, _P, _P, _P, _P, _I, _I, _F, _P], _I),
    "gdn_decode_linear_splits": ([_I, _L, _L], _I),
    "gdn_decode_linear_packed_partial": ([_P, _L, _P, _P, _I, _L, _L, _L, _P], _I),
    "gdn_add_rmsnorm_partial": ([_P, _P, _I, _P, _P, _P, _I, _I, _F, _P], _I),
    "gdn_swiglu_partial": ([_P, _I, _P, _I, _L, _P], _I),
    "gdn_attn_decode_workspace_bytes": ([_I, _I, _I, _I], _L),
    "gdn_attn_decode": ([_P, _L, _P, _P, _P, _P, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I, _F, _P], _I),
    "gdn_attn_decode_partial": ([_P, _I, _P, _P, _P, _P, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _I, _I, _F, _P],
                                _I),
    "gdn_conv_prefill": ([_P, _L, _P, _P, _P, _P, _P, _L, _P, _I, _I, _I, _I, _P], _I),
    "gdn_gating": ([_P, _P, _L, _P, _P, _P, _P, _L, _I, _P], _I),
    "gdn_decode_fused_masked": ([_P, _L, _P, _L, _P, _P, _L, _P, _P, _P, _P, _P, _P, _I, _F, _P, _P, _P, _I,
                                 _I, _I, _I, _I, _P], _I),
    "gdn_chunk_prefill_rows": ([_P, _L, _P, _L, _P, _L, _P, _P, _I, _P, _P, _P, _I, _P, _L, _P, _P, _L, _I,
                                _I, _I, _I, _I, _I, _I, _P, _L, _P], _I),
    "gdn_chunk_prefill_rows_gated": ([_P, _L, _P, _L, _P, _L, _P, _P, _I, _P, _P, _P, _I, _P, _L, _P, _P, _L,
                                      _I, _I, _I, _I, _I, _I, _I, _P, _L, _P, _I, _F, _P, _L, _P], _I),
    "gdn_prefill_layer_rows": ([_P, _L, _P, _L, _P, _P, _L, _P, _P, _P, _P, _P, _I, _F, _P, _P, _P, _P, _P, _I,
                                _P, _L, _P, _P, _L, _I, _I, _I, _I, _I, _I, _P, _L, _P], _I),
    "gdn_chunk_prefill_noalloc": ([_P, _L, _P, _L, _P, _L, _P, _P, _I, _P, _P, _P, _I, _P, _L, _P, _P, _L, _I,
                                   _I, _I, _I, _I, _I, _I, _P], _I),
    "gdn_conv_prefill_rows": ([_P, _L, _P, _P, _P, _P, _P, _P, _I, _L, _P, _I, _I, _I, _I, _P], _I),
    "gdn_chunk_prefill_inverse": ([_P, _L, _P, _P, _I, _L, _P, _P, _L, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P,
                                   _L, _P], _I),
    "gdn_chunk_prefill_generic": ([_P, _L, _P, _L, _P, _L, _P, _P, _I, _P, _P, _P, _I, _P, _L, _P, _I, _I, _I,
                                   _I, _I, _I, _I, _I, _P], _I),
}

_lib = None


class GDNError(RuntimeError):
    """A C-ABI call of the HIP library returned an error code."""


def lib():
    """Load the library once (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GDNError(f"{LIB_PATH} is missing: build it first (__graft_entry__.build() or "
                           f"python -m <package>.build); there is no CPU fallback")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name, None)
            if fn is None:
                continue
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def exported_symbols():
    """Names from the signature table that the loaded library exports."""
    h = lib()
    return [n for n in _SIGNATURES if getattr(h, n, None) is not None]


def call(name, *args):
    """Call a C-ABI entry point; raise GDNError with the library's message on failure."""
    fn = getattr(lib(), name)
    rc = fn(*args)
    if rc != 0:
        msg = lib().gdn_last_error().decode(errors="replace")
        raise GDNError(f"{name} failed (code {rc}): {msg}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t):
    """Raw hipStream_t of torch's current stream on t's device (torch's raw-handle query when it has
    one: no Stream object per call)."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(t.get_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def ptr_int(t):
    """Device address as a plain int (None for None): what a c_void_p argument takes directly."""
    return None if t is None else t.data_ptr()


def dtype_code(t):
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float16:
        return F16
    raise TypeError(f"unsupported dtype {t.dtype} (float32, bfloat16 or float16)")


def dense_rows(t):
    """A 2-D [rows, cols] tensor as the row kernels read it: unit column stride, row stride a multiple
    of 8 elements, base 16-byte aligned -- t itself when it qualifies, else a dense copy.  Returns
    (tensor, row stride).  torch gives a size-1 dimension an arbitrary stride, and one row's stride
    is never used, so a single row counts its length as its stride."""
    rs = t.stride(0) if t.shape[0] > 1 else t.shape[1]
    if (t.stride(1) != 1 and t.shape[1] > 1) or rs % 8 or t.data_ptr() % 16:
        t = t.clone(memory_format=torch.contiguous_format)
        rs = t.shape[1]
    return t, rs


def require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("GDN HIP ops need tensors on a ROCm GPU device (no CPU fallback)")
