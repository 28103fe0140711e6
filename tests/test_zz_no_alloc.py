"""The allocation-free chunked prefill entry point (gdn_chunk_prefill_noalloc, static per-device
scratch) against the workspace entry point (gdn_chunk_prefill_rows) through the C ABI: two calls
in a row, the second smaller, each bit-identical (the same kernels on the same inputs); a request
beyond the scratch is refused before any launch; one call captured in a HIP graph and replayed,
each replay bit-identical to the workspace entry point."""
import importlib

import pytest
import torch

from conftest import PKG_NAME

CHUNK = 64


def _inputs(lens, Hk, Hv, seed, D=128):
    g_ = torch.Generator().manual_seed(seed)
    T = sum(lens)
    bf = torch.bfloat16
    q = torch.randn(T, Hk, D, generator=g_).to(bf)
    k = torch.randn(T, Hk, D, generator=g_).to(bf)
    v = torch.randn(T, Hv, D, generator=g_).to(bf)
    beta = torch.sigmoid(torch.randn(T, Hv, generator=g_)).to(bf)
    g = -torch.nn.functional.softplus(torch.randn(T, Hv, generator=g_) + 2) * 0.1
    s0 = 0.02 * torch.randn(len(lens), Hv, D, D, generator=g_)
    return q, k, v, g, beta, s0


def _call(L, name, q, k, v, g, beta, s0, cu, chunk0, total_chunks, Hk, Hv, work=None):
    T, D, nseq = q.shape[0], q.shape[2], s0.shape[0]
    out = torch.empty(T, Hv, D, dtype=torch.bfloat16, device=q.device)
    fin = torch.empty_like(s0)
    args = [L.ptr(q), q.stride(0), L.ptr(k), k.stride(0), L.ptr(v), v.stride(0), L.ptr(g), L.ptr(beta), L.BF16,
            L.ptr(s0), L.ptr(fin), None, nseq, L.ptr(out), T, L.ptr(cu), L.ptr(chunk0), total_chunks, nseq, 0, Hk,
            Hv, D, L.BF16, 1]
    if work is not None:
        args += [L.ptr(work), work.numel()]
    L.call(name, *args, L.stream_of(q))
    return out, fin


@pytest.mark.gpu
def test_noalloc_prefill_matches_workspace_entry_point(gdn, dev):
    L = importlib.import_module(PKG_NAME + "._lib")
    cases = [([300, 1, 257, 130], 4, 8, 80),   # 4 packed sequences, 13 chunks x 8 heads
             ([150], 2, 4, 81)]                # then a smaller call: 3 chunks x 4 heads
    for lens, Hk, Hv, seed in cases:
        q, k, v, g, beta, s0 = (x.to(dev) for x in _inputs(lens, Hk, Hv, seed))
        cu_h = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
        nch = [(n + CHUNK - 1) // CHUNK for n in lens]
        c0_h = torch.tensor([0] + list(torch.cumsum(torch.tensor(nch), 0)), dtype=torch.int32)
        total = int(c0_h[-1])
        cu, c0 = cu_h.to(dev), c0_h.to(dev)
        wbytes = int(L.lib().gdn_chunk_prefill_workspace_bytes(total, len(lens), Hv))
        assert wbytes <= 256 << 20
        work = torch.empty(wbytes, dtype=torch.uint8, device=dev)
        o_ref, f_ref = _call(L, "gdn_chunk_prefill_rows", q, k, v, g, beta, s0, cu, c0, total, Hk, Hv, work=work)
        o, f = _call(L, "gdn_chunk_prefill_noalloc", q, k, v, g, beta, s0, cu, c0, total, Hk, Hv)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(f, f_ref), f"lens {lens}"
    # beyond the scratch (10.5 KiB of inverse records per (chunk, value head)): refused on the host
    # before any launch
    with pytest.raises(L.GDNError, match="static scratch holds"):
        _call(L, "gdn_chunk_prefill_noalloc", q, k, v, g, beta, s0, cu, c0, 20_000, Hk, Hv)


@pytest.mark.gpu
def test_noalloc_prefill_under_graph_capture(gdn, dev):
    """The entry point is for callers under HIP graph capture: capture one call (on torch's capture
    stream), replay it three times with eager work and a synchronisation between the replays, and
    require every replay to equal the workspace entry point's result bit for bit."""
    L = importlib.import_module(PKG_NAME + "._lib")
    lens, Hk, Hv = [300, 1, 257, 130], 4, 8
    q, k, v, g, beta, s0 = (x.to(dev) for x in _inputs(lens, Hk, Hv, 90))
    cu_h = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    nch = [(n + CHUNK - 1) // CHUNK for n in lens]
    c0_h = torch.tensor([0] + list(torch.cumsum(torch.tensor(nch), 0)), dtype=torch.int32)
    total = int(c0_h[-1])
    cu, c0 = cu_h.to(dev), c0_h.to(dev)
    work = torch.empty(int(L.lib().gdn_chunk_prefill_workspace_bytes(total, len(lens), Hv)), dtype=torch.uint8,
                       device=dev)
    o_ref, f_ref = _call(L, "gdn_chunk_prefill_rows", q, k, v, g, beta, s0, cu, c0, total, Hk, Hv, work=work)
    T, D = q.shape[0], q.shape[2]
    out = torch.empty(T, Hv, D, dtype=torch.bfloat16, device=dev)
    fin = torch.empty_like(s0)
    args = [L.ptr(q), q.stride(0), L.ptr(k), k.stride(0), L.ptr(v), v.stride(0), L.ptr(g), L.ptr(beta), L.BF16,
            L.ptr(s0), L.ptr(fin), None, len(lens), L.ptr(out), T, L.ptr(cu), L.ptr(c0), total, len(lens), 0, Hk,
            Hv, D, L.BF16, 1]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            L.call("gdn_chunk_prefill_noalloc", *args, L.stream_of(q))
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        fin.zero_()
        # other work on the same scratch between replays: an eager call of the entry point itself
        o_e, f_e = _call(L, "gdn_chunk_prefill_noalloc", q, k, v, g, beta, s0, cu, c0, total, Hk, Hv)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, o_ref) and torch.equal(fin, f_ref), f"replay {i}"
        assert torch.equal(o_e, o_ref) and torch.equal(f_e, f_ref), f"eager call {i}"
