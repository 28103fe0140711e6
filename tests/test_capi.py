"""CPU checks of the C-ABI library: it loads, exports every entry point include/gdn_mi355x.h
declares, and rejects bad arguments with an error code and message before touching a GPU."""
import ctypes
import importlib
import os
import re

import pytest

from conftest import PKG_NAME, ROOT

HEADER = os.path.join(ROOT, "include", "gdn_mi355x.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\*?\s+\*?(gdn_[a-z0-9_]+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    return importlib.import_module(PKG_NAME + "._lib")


def test_header_declares_entry_points():
    syms = declared_symbols()
    for name in ("gdn_recurrent_step", "gdn_conv_update", "gdn_gated_rmsnorm", "gdn_decode_fused",
                 "gdn_chunk_prefill", "gdn_conv_prefill", "gdn_gating", "gdn_unit_lower_inv",
                 "gdn_decode_fused_masked", "gdn_chunk_prefill_rows", "gdn_conv_prefill_rows",
                 "gdn_decode_linear", "gdn_decode_linear_workspace_bytes", "gdn_decode_linear_pack",
                 "gdn_decode_linear_packed", "gdn_add_rmsnorm", "gdn_chunk_prefill_rows_gated",
                 "gdn_prefill_layer_rows", "gdn_prefill_layer_workspace_bytes", "gdn_chunk_prefill_noalloc",
                 "gdn_chunk_prefill_generic", "gdn_chunk_prefill_inverse"):
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    handle = lib.lib()
    missing = [s for s in declared_symbols() if getattr(handle, s, None) is None]
    assert not missing, f"declared but not exported: {missing}"
    bound = set(lib.exported_symbols())
    assert set(declared_symbols()) <= bound, "every declared entry point has a ctypes signature"


def test_version_limits_and_error_path(lib):
    h = lib.lib()
    assert h.gdn_version() >= 100
    d, r, k = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert h.gdn_limits(ctypes.byref(d), ctypes.byref(r), ctypes.byref(k)) == 0
    assert d.value == 128 and r.value >= 3 and k.value >= 4
    # argument validation runs on the host, before any HIP call
    rc = h.gdn_recurrent_step(None, 0, None, 0, None, 0, None, None, 1, None, None, None,
                              1, 1, 1, 128, 1, 1, None)
    assert rc == 1 and b"null" in h.gdn_last_error()
    rc = h.gdn_conv_update(ctypes.c_void_p(16), 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None,
                           ctypes.c_void_p(16), 0, 1, 8, 9, None)
    assert rc == 2 and b"kernel size" in h.gdn_last_error()
    p = ctypes.c_void_p(256)
    rc = h.gdn_decode_fused(p, 0, p, 0, p, p, 0, p, p, None, p, p, p, 1, ctypes.c_float(1e-6), p, p,
                            1, 16, 32, 64, 4, None)
    assert rc == 2 and b"head dim" in h.gdn_last_error()
    rc = h.gdn_decode_fused_masked(p, 0, p, 0, p, p, 0, p, p, None, p, p, p, 1, ctypes.c_float(1e-6), p, p,
                                   None, 1, 16, 32, 64, 4, None)
    assert rc == 2 and b"head dim" in h.gdn_last_error()
    # without state_rows the slot-row variants need n_rows == nseq
    rc = h.gdn_chunk_prefill_rows(p, 0, p, 0, p, 0, p, p, 1, None, None, None, 3, p, 64, None, None, 1, 2, 32,
                                  16, 32, 128, 1, 1, p, 1 << 30, None)
    assert rc == 1 and b"n_rows" in h.gdn_last_error()
    rc = h.gdn_conv_prefill_rows(p, 8, p, None, None, p, None, None, 5, 8, None, 1, 8, 8, 4, None)
    assert rc == 1 and b"n_rows" in h.gdn_last_error()
    # the scan copies 16-byte pieces of initial states: states must be 16-byte aligned
    rc = h.gdn_chunk_prefill(p, 0, p, 0, p, 0, p, p, 1, ctypes.c_void_p(256 + 4), None, p, 64, None, None, 1, 1,
                             64, 16, 32, 128, 1, 1, p, 1 << 30, None)
    assert rc == 1 and b"16-byte" in h.gdn_last_error()
    # decode projections: at most 16 rows, K a multiple of 128, packed size = padded rows x K
    rc = h.gdn_decode_linear(p, 256, p, 256, p, 256, 17, 256, 256, None, 0, None)
    assert rc == 2 and b"rows" in h.gdn_last_error()
    rc = h.gdn_decode_linear(p, 256, p, 256, p, 256, 16, 256, 100, None, 0, None)
    assert rc == 2 and b"multiple" in h.gdn_last_error()
    rc = h.gdn_decode_linear_packed(p, 256, p, p, 256, 16, 256, 100, None, 0, None)
    assert rc == 2 and b"multiple" in h.gdn_last_error()
    assert h.gdn_decode_linear_workspace_bytes(16, 248320, 5120) == 0
    small = h.gdn_decode_linear_workspace_bytes(16, 5120, 17408)
    assert small > 0 and small % (16 * 5120 * 4) == 0
    rc = h.gdn_decode_linear(p, 17408, p, 17408, p, 5120, 16, 5120, 17408, None, 0, None)
    assert rc == 1 and b"workspace" in h.gdn_last_error()
    assert h.gdn_decode_linear_packed_elems(98, 256) == 112 * 256
    assert h.gdn_decode_linear_packed_elems(98, 100) == 0
    rc = h.gdn_add_rmsnorm(p, p, p, None, p, 4, 256, ctypes.c_float(1e-6), None)
    assert rc == 1 and b"null" in h.gdn_last_error()
    need = h.gdn_chunk_prefill_workspace_bytes(10, 1, 32)
    assert need > 0 and need % 256 == 0
    # the generic chunked rule: head dims 16 / 32 / 64 / 128 only, a known dtype, consistent sizes
    rc = h.gdn_chunk_prefill_generic(p, 256, p, 256, p, 256, p, p, 0, None, None, None, 1, p, 64, None, 1, 64, 2,
                                     2, 96, 64, 0, 1, None)
    assert rc == 2 and b"d_k 96" in h.gdn_last_error()
    rc = h.gdn_chunk_prefill_generic(p, 256, p, 256, p, 256, p, p, 0, None, None, None, 1, p, 64, None, 1, 64, 2,
                                     2, 64, 64, 7, 1, None)
    assert rc == 1 and b"dtype" in h.gdn_last_error()
    rc = h.gdn_chunk_prefill_generic(p, 256, p, 256, p, 256, p, p, 0, None, None, None, 1, p, 65, None, 1, 64, 2,
                                     2, 64, 64, 0, 1, None)
    assert rc == 1 and b"nseq*seq_len" in h.gdn_last_error()
    # gdn_chunk_prefill hands other dtypes and head dims to the generic rule (whose checks then run)
    rc = h.gdn_chunk_prefill(p, 0, p, 0, p, 0, p, p, 1, None, None, p, 64, None, None, 1, 1, 64, 16, 32, 96, 0, 1,
                             p, 1 << 30, None)
    assert rc == 2 and b"gdn_chunk_prefill_generic: d_k 96" in h.gdn_last_error()
    # the inverse kernel alone: bf16 keys at D = 128 only, and a workspace
    rc = h.gdn_chunk_prefill_inverse(p, 256, p, p, 1, 64, None, None, 1, 1, 64, 2, 2, 64, 1, 1, p, None, p, 1 << 30,
                                     None)
    assert rc == 2 and b"D = 128" in h.gdn_last_error()
    rc = h.gdn_chunk_prefill_inverse(p, 256, p, p, 1, 64, None, None, 1, 1, 64, 2, 2, 128, 1, 1, p, None, p, 16,
                                     None)
    assert rc == 1 and b"workspace" in h.gdn_last_error()
    with pytest.raises(lib.GDNError):
        lib.call("gdn_gated_rmsnorm", None, 0, None, 0, None, 1, None, 1, 128, ctypes.c_float(1e-6), None)



def test_prefill_layer_entry_host_checks(lib):
    """gdn_prefill_layer_rows validates on the host before any HIP call: its workspace holds the conv
    output, beta and g besides the chunked rule's workspace; null pointers, an unsupported head dim,
    misaligned gate rows and a short workspace are refused with their codes."""
    h = lib.lib()
    T, nch, nseq, Hk, Hv, D, K = 1000, 20, 2, 16, 32, 128, 4
    C = (2 * Hk + Hv) * D
    need = h.gdn_prefill_layer_workspace_bytes(T, nch, nseq, Hk, Hv, D)
    assert need % 256 == 0
    assert need >= T * C * 2 + T * Hv * 2 + T * Hv * 4 + h.gdn_chunk_prefill_workspace_bytes(nch, nseq, Hv)
    p = ctypes.c_void_p(256)
    eps = ctypes.c_float(1e-6)

    def call(mixed=p, z=p, D_=D, ws=need, z_stride=Hv * D, n_rows=nseq, cu=p, chunk0=p, seq_len=0, nch_=nch):
        return h.gdn_prefill_layer_rows(mixed, C, z, z_stride, p, p, Hv, p, None, p, p, p, 1, eps, None, p, None, p,
                                        None, n_rows, p, T, cu, chunk0, nch_, nseq, seq_len, Hk, Hv, D_, K, p, ws, None)

    assert call(mixed=None) == 1 and b"null" in h.gdn_last_error()
    assert call(D_=64) == 2 and b"head dim" in h.gdn_last_error()
    assert call(z=ctypes.c_void_p(256 + 2)) == 1 and b"gate rows" in h.gdn_last_error()
    assert call(z_stride=Hv * D - 8) == 1 and b"gate rows" in h.gdn_last_error()
    assert call(n_rows=nseq + 1) == 1 and b"n_rows" in h.gdn_last_error()
    assert call(ws=need - 256) == 1 and b"workspace" in h.gdn_last_error()
    # the chunked rule's own checks run before the prologue launch (which would already overwrite the
    # conv state): packed sequences without their chunk table, a uniform batch whose chunk count does
    # not match its length -- refused on the host, no launch (a launch would fail here: no GPU)
    assert call(chunk0=None) == 1 and b"seq_chunk0" in h.gdn_last_error()
    assert call(cu=None, chunk0=None, seq_len=T // nseq) == 1 and b"total_chunks" in h.gdn_last_error()
