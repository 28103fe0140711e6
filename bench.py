"""Benchmark of the GDN hot path on one MI355X.

Default workload (the headline line): the 16-slot GDN decode step over 48 layers -- per layer the
fused conv update + SiLU + gating + l2norm + recurrent fp32 state read-modify-write + gated RMSNorm
for 16 slots x 1 token, H_k=16, H_v=32, d=128, conv channels 8192, kernel 4 -- with 48 DISTINCT
layer states (3.2 GB working set, so the 256 MB Infinity Cache cannot serve them), captured once as
a HIP graph and replayed.  A "step" is one replay (48 layers).  ``value`` is microseconds per layer.

Also reported (``secondary``): the decode layer at one TP=2 rank's share of the heads (H_k=8,
H_v=16); chunked GDN prefill at T=8192 (B=1, H_k=16, H_v=32, d=128, bf16 inputs, fp32 state) in
tokens/s/layer with its bf16-MFMA and HBM fractions, the fused varlen prefill layer, T=32768, the
chunked rule at Qwen3.5-27B's GDN shape (H_k=16, H_v=48) at T=8192 and 353 tokens, T=8192 at slow
decay (g ~ -0.002 a token: the exact segment path), and whole decode steps at Qwen3.5-27B shape (the
hybrid 64-layer stack, and its 48 GDN layers with projections) in tokens/s.  CPU baselines (the
oracle on the host's cores; warm-up, then the median of 5 passes) for the decode step, T=8192, the
varlen layer and T=32768.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill]
                      [--only decode|prefill|prefill8192|varlen|hybrid|attention]
"""
import argparse
import importlib
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
PKG = "910b_e2e_accleration_by_codex_amd"

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15         # flop/s, dense bf16 MFMA

N_SLOTS, HK, HV, D, KC, LAYERS = 16, 16, 32, 128, 4, 48
# HBM bytes per decode_fused_kernel launch at this workload, measured with two rocprofv3 --pmc runs
# (FETCH_SIZE, WRITE_SIZE) scaled by what the counters read for a 256 MiB device copy
DECODE_TRAFFIC = 69_993_300
C = (2 * HK + HV) * D


def decode_bytes_per_layer(hk=HK, hv=HV):
    """Algorithmic HBM bytes of one fused decode layer (each tensor touched once)."""
    c = (2 * hk + hv) * D
    state = 2 * N_SLOTS * hv * D * D * 4            # fp32 state read + write
    conv = 2 * N_SLOTS * c * KC * 2                 # bf16 conv state read + write
    conv_w = c * KC * 2
    mixed = N_SLOTS * c * 2
    z = N_SLOTS * hv * D * 2
    out = N_SLOTS * hv * D * 2
    ab = 2 * N_SLOTS * hv * 2
    params = hv * 4 * 2 + D * 2                     # A_log, dt_bias fp32; norm weight bf16
    return state + conv + conv_w + mixed + z + out + ab + params


def make_decode_layers(dev, seed=0, hk=HK, hv=HV):
    g_ = torch.Generator(device="cpu").manual_seed(seed)
    c = (2 * hk + hv) * D
    layers = []
    for _ in range(LAYERS):
        layers.append(dict(
            mixed=torch.randn(N_SLOTS, c, generator=g_).to(torch.bfloat16).to(dev),
            z=torch.randn(N_SLOTS, hv * D, generator=g_).to(torch.bfloat16).to(dev),
            a=torch.randn(N_SLOTS, hv, generator=g_).to(torch.bfloat16).to(dev),
            b=torch.randn(N_SLOTS, hv, generator=g_).to(torch.bfloat16).to(dev),
            conv_state=torch.randn(N_SLOTS, c, KC, generator=g_).to(torch.bfloat16).to(dev),
            conv_weight=(0.5 * torch.randn(c, KC, generator=g_)).to(torch.bfloat16).to(dev),
            A_log=torch.full((hv,), -2.302585092994046, device=dev),   # log(0.1)
            dt_bias=torch.full((hv,), 2.0, device=dev),
            norm_weight=(1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16).to(dev),
            rec_state=(0.02 * torch.randn(N_SLOTS, hv, D, D, generator=g_)).to(dev),
        ))
    return layers


def decode_step(gdn, layers, outs, hk=HK, hv=HV):
    for p, o in zip(layers, outs):
        gdn.gdn_decode_core(p["mixed"], p["z"], p["a"], p["b"], p["conv_state"], p["conv_weight"],
                            p["A_log"], p["dt_bias"], p["norm_weight"], p["rec_state"], hk, hv, D,
                            out=o)
    return outs


def bench_decode(gdn, dev, steps, warmup, hk=HK, hv=HV):
    layers = make_decode_layers(dev, hk=hk, hv=hv)
    outs = [torch.empty(N_SLOTS, hv * D, dtype=torch.bfloat16, device=dev) for _ in range(LAYERS)]
    graph = gdn.GDNDecodeGraph(lambda: decode_step(gdn, layers, outs, hk, hv), device=dev)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    # HIP events on the stream the graph's kernels run on (the current stream at replay)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    us_layer = ms * 1000.0 / LAYERS
    # eager (non-graph) back-to-back launches of the same kernel, for the per-launch duration
    e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e2.record(stream)
    for _ in range(steps):
        decode_step(gdn, layers, outs, hk, hv)
    e3.record(stream)
    torch.cuda.synchronize()
    us_eager = e2.elapsed_time(e3) * 1000.0 / (steps * LAYERS)
    return dict(ms_per_step=ms, us_per_layer=us_layer, us_per_layer_eager=us_eager, wall_s=wall)


def bench_decode_tp_share(gdn, dev, steps, warmup, tp=2):
    """The decode layer at one tensor-parallel rank's share of the heads (H_k/tp, H_v/tp: the slicing
    of src/cb_tp.py:69-97); the all-reduce after out_proj that a multi-GPU step adds is not here."""
    hk, hv = HK // tp, HV // tp
    r = bench_decode(gdn, dev, steps, warmup, hk=hk, hv=hv)
    b = decode_bytes_per_layer(hk, hv)
    return dict(workload=f"decode layer at one TP={tp} rank's share: 16 slots, H_k={hk} H_v={hv} d={D}, conv "
                         f"{(2 * hk + hv) * D}x{KC}, 48 distinct layers, graph replay (the all-reduce after "
                         f"out_proj not included)",
                us_per_layer=round(r["us_per_layer"], 3), hbm_frac=round(b / (r["us_per_layer"] * 1e-6) / HBM_PEAK, 4),
                bytes=b)


def prefill_flops(T, hv=HV, d=D, chunk=64):
    """Algorithmic flops of the chunked rule: 10*C*d + 6*d^2 per token per value head (the eight
    contractions of one chunk; inverse and elementwise work excluded)."""
    return T * hv * (10 * chunk * d + 6 * d * d)


def prefill_bytes(T, nseq=1, hk=HK, hv=HV, d=D):
    """Core kernel HBM bytes: q, k (unrepeated) + v in, out, g fp32 + beta bf16, initial + final state."""
    per_tok = 2 * (2 * hk * d) + 2 * hv * d + 6 * hv + 2 * hv * d
    return T * per_tok + nseq * 2 * hv * d * d * 4


def prefill_layer_bytes(T, nseq, hv=HV, d=D, c=C, k=KC):
    """Fused layer bytes: mixed_qkv in (C channels) + z + a, b + normed out, states, conv states."""
    per_tok = 2 * c + 2 * hv * d + 4 * hv + 2 * hv * d
    return T * per_tok + nseq * (2 * hv * d * d * 4 + c * k * 2)


def _time(fn, reps, dev):
    """GPU time per call with the host enqueueing ahead (as a serving loop does): a spin kernel of
    ~20 ms keeps the GPU busy while the timed calls are queued, so the event window holds only
    their GPU work, not the host's time to issue the first call."""
    fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(50_000_000)
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / reps


def _gdn_inputs(T, seed, dev, nseq=1, hk=HK, hv=HV, decay=0.1):
    g_ = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(1, T, hk, D, generator=g_).to(torch.bfloat16).to(dev)
    k = torch.randn(1, T, hk, D, generator=g_).to(torch.bfloat16).to(dev)
    v = torch.randn(1, T, hv, D, generator=g_).to(torch.bfloat16).to(dev)
    beta = torch.sigmoid(torch.randn(1, T, hv, generator=g_)).to(torch.bfloat16).to(dev)
    g = (-torch.nn.functional.softplus(torch.randn(1, T, hv, generator=g_) + 2) * decay).to(dev)
    s0 = (0.02 * torch.randn(nseq, hv, D, D, generator=g_)).to(dev)
    return q, k, v, g, beta, s0


def _fractions(name, us, F, B, tokens):
    return dict(workload=name, us_per_layer=round(us, 2), tokens_per_s_per_layer=round(tokens / (us * 1e-6)),
                mfma_frac=round(F / (us * 1e-6) / BF16_PEAK, 4), hbm_frac=round(B / (us * 1e-6) / HBM_PEAK, 4),
                flops=F, bytes=B)


def bench_prefill(gdn, dev, T=8192, reps=5, seed=0, hk=HK, hv=HV, note=None, decay=0.1):
    """Chunked rule alone, B=1, T tokens, hk key heads read by hv value heads (value head h reads key
    head h // (hv / hk)); g = -softplus(N(0, 1) + 2) * decay per token."""
    q, k, v, g, beta, s0 = _gdn_inputs(T, seed, dev, hk=hk, hv=hv, decay=decay)
    us = _time(lambda: gdn.fast_chunk_gated_delta_rule_v2(q, k, v, g, beta, initial_state=s0, output_final_state=True,
                                                          use_qk_l2norm_in_kernel=True), reps, dev)
    slow = "" if decay == 0.1 else f" g~-{2.1 * decay:g}/token"
    res = _fractions(f"chunked rule B=1 T={T} H_k={hk} H_v={hv} d={D} bf16{slow}", us, prefill_flops(T, hv=hv),
                     prefill_bytes(T, hk=hk, hv=hv), T)
    if note:
        res["note"] = note
    return res


def _varlen_inputs(seed=2):
    """16 packed prompts with lengths uniform in [200, 1500] (seeded), the layer's weights and states."""
    g_ = torch.Generator(device="cpu").manual_seed(seed)
    lens = torch.randint(200, 1501, (16,), generator=g_)
    cu = torch.zeros(17, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    T = int(cu[-1])
    x = dict(mixed=torch.randn(T, C, generator=g_).to(torch.bfloat16),
             z=torch.randn(T, HV * D, generator=g_).to(torch.bfloat16),
             a=torch.randn(T, HV, generator=g_).to(torch.bfloat16),
             b=torch.randn(T, HV, generator=g_).to(torch.bfloat16),
             cw=(0.5 * torch.randn(C, KC, generator=g_)).to(torch.bfloat16),
             A_log=torch.full((HV,), -2.302585092994046), dt=torch.full((HV,), 2.0),
             nw=(1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16),
             s0=0.02 * torch.randn(16, HV, D, D, generator=g_))
    return cu, T, x


def bench_prefill_varlen(gdn, dev, reps=5, seed=2, cpu=False, cpu_reps=5):
    """Fused prefill layer (conv1d prefill + SiLU, l2norm, gating, chunked rule, gated RMSNorm) over
    16 packed prompts with lengths uniform in [200, 1500], random initial states, zero conv history.
    With cpu: the oracle's layer (its per-sequence loop, as the reference runs one sequence per call)
    on the host's cores, warm-up then the median of cpu_reps passes, as the CPU baseline."""
    cu, T, x = _varlen_inputs(seed)
    d = {n: t.to(dev) for n, t in x.items()}
    # lengths on the host, as a scheduler holds them: the batch's sequence table is checked and uploaded
    # once per batch step (it is the same for every layer), outside the timed layer calls
    table = gdn.Varlen(cu, T, dev)
    us = _time(lambda: gdn.gdn_prefill_core(d["mixed"], d["z"], d["a"], d["b"], d["cw"], d["A_log"], d["dt"],
                                            d["nw"], HK, HV, D, cu_seqlens=table, initial_state=d["s0"]), reps, dev)
    res = _fractions(f"fused prefill layer, 16 packed prompts ({T} tokens), H_k={HK} H_v={HV} d={D}", us,
                     prefill_flops(T), prefill_layer_bytes(T, 16), T)
    res["note"] = ("the batch's Varlen table (host checks + one pinned upload) is built once per batch step "
                   "outside the timed layer calls")
    if cpu:
        oracle = importlib.import_module("oracle.gdn_oracle")
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        dt = _median_time(lambda: oracle.gdn_prefill_core(x["mixed"], x["z"], x["a"], x["b"], x["cw"], x["A_log"],
                                                          x["dt"], x["nw"], HK, HV, D, cu_seqlens=cu,
                                                          initial_state=x["s0"]), cpu_reps)
        model = cpu_model()
        res["cpu_baseline"] = dict(value=round(T / dt), unit="tokens/s/layer", us_per_layer=round(dt * 1e6),
                                   cores=threads, kind="port", cpu_model=model,
                                   sample=f"oracle gdn_prefill_core (per-sequence loop) on the same 16 prompts "
                                          f"({T} tokens), warm-up then median of {cpu_reps} passes, torch "
                                          f"{torch.__version__} CPU, {threads} threads on {model}")
    return res


def bench_prefill_long(gdn, dev, T=32768, seed=3, check=True, cpu_reps=5):
    """B=1, T=32768: per-layer time and the final-state rel-L2 against the CPU oracle; the oracle's
    pass, timed, is also the CPU baseline (median of cpu_reps after the checking pass)."""
    q, k, v, g, beta, s0 = _gdn_inputs(T, seed, dev)
    run = lambda: gdn.fast_chunk_gated_delta_rule_v2(q, k, v, g, beta, initial_state=s0, output_final_state=True,
                                                     use_qk_l2norm_in_kernel=True)
    us = _time(run, 2, dev)
    res = _fractions(f"chunked rule B=1 T={T} H_k={HK} H_v={HV} d={D} bf16", us, prefill_flops(T),
                     prefill_bytes(T), T)
    if check:
        oracle = importlib.import_module("oracle.gdn_oracle")
        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        o, s = run()
        r = HV // HK
        oc = lambda x: x.cpu().repeat_interleave(r, dim=2)
        args = (oc(q), oc(k), v.cpu(), g.cpu(), beta.cpu(), 64, s0.cpu(), True, True)
        o_ref, s_ref = oracle.chunk_gated_delta_rule_v2(*args)
        rel = lambda x, y: ((x.double().cpu() - y.double()).norm() / y.double().norm()).item()
        res["out_rel_l2_vs_oracle"] = rel(o, o_ref)
        res["state_rel_l2_vs_oracle"] = rel(s, s_ref)
        del o_ref, s_ref
        # the checking pass doubles as the warm-up; then the median of `cpu_reps` timed passes
        dt = _median_time(lambda: oracle.chunk_gated_delta_rule_v2(*args), cpu_reps, warm=False)
        model = cpu_model()
        res["cpu_baseline"] = dict(value=round(T / dt), unit="tokens/s/layer", us_per_layer=round(dt * 1e6),
                                   cores=threads, kind="port", cpu_model=model,
                                   sample=f"oracle chunk_gated_delta_rule_v2, B=1 T={T} H_v={HV} d={D}, median of "
                                          f"{cpu_reps} passes after the one that checks the GPU result, torch "
                                          f"{torch.__version__} CPU, {threads} threads on {model}")
    return res


def cpu_model():
    """The host CPU's model name (first /proc/cpuinfo entry), for the baseline record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, reps, warm=True):
    """One untimed warm-up pass (unless the caller has just run one), then the median wall time of
    `reps` passes."""
    if warm:
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline_prefill(T=8192, seed=0, reps=5):
    """The oracle's chunked rule (torch CPU restatement of src/gdn_chunk_fast2.py) at T=8192: one
    warm-up pass, then the median of `reps` passes."""
    oracle = importlib.import_module("oracle.gdn_oracle")
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    q, k, v, g, beta, s0 = _gdn_inputs(T, seed, "cpu")
    r = HV // HK
    q, k = q.repeat_interleave(r, 2), k.repeat_interleave(r, 2)
    dt = _median_time(lambda: oracle.chunk_gated_delta_rule_v2(q, k, v, g, beta, 64, s0, True, True), reps)
    model = cpu_model()
    return dict(value=round(T / dt), unit="tokens/s/layer", us_per_layer=round(dt * 1e6), cores=threads,
                kind="port", cpu_model=model,
                sample=f"oracle chunk_gated_delta_rule_v2, B=1 T={T} H_v={HV} d={D}, warm-up then median of "
                       f"{reps} passes, torch {torch.__version__} CPU, {threads} threads on {model}")


def cpu_baseline_decode(layers_cpu=LAYERS, reps=5):
    """The oracle (torch CPU restatement of the reference decode path) on this host's cores."""
    oracle = importlib.import_module("oracle.gdn_oracle")
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g_ = torch.Generator().manual_seed(1)
    ls = []
    for _ in range(layers_cpu):
        ls.append(dict(
            mixed=torch.randn(N_SLOTS, C, generator=g_).to(torch.bfloat16),
            z=torch.randn(N_SLOTS, HV * D, generator=g_).to(torch.bfloat16),
            a=torch.randn(N_SLOTS, HV, generator=g_).to(torch.bfloat16),
            b=torch.randn(N_SLOTS, HV, generator=g_).to(torch.bfloat16),
            conv_state=torch.randn(N_SLOTS, C, KC, generator=g_).to(torch.bfloat16),
            conv_weight=(0.5 * torch.randn(C, KC, generator=g_)).to(torch.bfloat16),
            A_log=torch.full((HV,), -2.302585092994046), dt_bias=torch.full((HV,), 2.0),
            norm_weight=(1 + 0.02 * torch.randn(D, generator=g_)).to(torch.bfloat16),
            rec_state=0.02 * torch.randn(N_SLOTS, HV, D, D, generator=g_)))

    def one():
        for p in ls:
            oracle.gdn_decode_core(p["mixed"], p["z"], p["a"], p["b"], p["conv_state"], p["conv_weight"],
                                   p["A_log"], p["dt_bias"], p["norm_weight"], p["rec_state"], HK, HV, D)
    us = _median_time(one, reps) * 1e6 / layers_cpu
    model = cpu_model()
    return dict(value=us, unit="us/layer", cores=threads, kind="port", cpu_model=model,
                sample=f"oracle gdn_decode_core, {layers_cpu} distinct layers per pass, warm-up then median "
                       f"of {reps} passes, same shapes as the GPU workload, torch {torch.__version__} CPU, "
                       f"{threads} threads on {model}")


def bench_attention(gdn, dev, reps=3, seed=4):
    """The decode attention of the hybrid stack's full-attention layers alone, at Qwen3.5-27B's
    attention shape: 16 slots, 24 q / 4 kv heads of 256, quarter rotary, positions = contexts uniform
    in [512, 4096].  Sixteen layers' KV caches are cycled so the cache reads come from HBM.  Bytes:
    each slot's K and V at positions 0..pos (the kernels' algorithmic reads)."""
    cb = importlib.import_module(PKG + ".cb_engine")
    nh, kv, hd, rd, T, L = 24, 4, 256, 64, 4112, 16
    g_ = torch.Generator().manual_seed(seed)
    ctx = torch.randint(512, 4097, (N_SLOTS,), generator=g_)
    bf = torch.bfloat16
    proj = torch.randn(N_SLOTS, (2 * nh + 2 * kv) * hd, generator=g_).to(bf).to(dev)
    qn = (0.1 * torch.randn(hd, generator=g_)).to(bf).to(dev)
    kn = (0.1 * torch.randn(hd, generator=g_)).to(bf).to(dev)
    inv = (1.0 / (10000.0 ** (torch.arange(0, rd, 2).float() / rd))).to(dev)
    kts = [torch.randn(N_SLOTS, kv, hd, T, device=dev).to(bf) for _ in range(L)]
    vcs = [torch.randn(N_SLOTS, kv, T, hd, device=dev).to(bf) for _ in range(L)]
    pos = ctx.to(dev)
    work = cb.attn_decode_workspace(N_SLOTS, nh, hd, T, dev)

    def layers():
        for i in range(L):
            cb.gqa_decode_attention(proj, pos, qn, kn, inv, kts[i], vcs[i], nh, kv, hd, rd, 1e-6, work=work)

    us = _time(layers, reps, dev) / L
    nbytes = int((ctx.double() + 1).sum()) * kv * hd * 2 * 2
    del kts, vcs
    torch.cuda.empty_cache()
    return {"workload": f"decode attention, 27B shape (24 q / 4 kv heads of 256), 16 slots, ctx U[512,4096] "
                        f"(mean {float(ctx.double().mean()):.1f})",
            "us_per_layer": round(us, 2), "kv_bytes_per_layer": nbytes,
            "hbm_frac": round(nbytes / (us * 1e-6) / HBM_PEAK, 4)}


def bench_hybrid(gdn, dev, steps=10, warmup=2, seed=4):
    """Whole decode steps at Qwen3.5-27B shape, 16 slots, contexts uniform in [512, 4096] with random
    GDN states and KV caches, HIP-graph replay (random-init bf16 weights):
      * the 64-layer hybrid stack (48 GDN + 16 GQA attention layers, SwiGLU MLPs, LM head 248320);
      * the 48 GDN layers alone with their projections (in_proj GEMM -> fused HIP core -> out_proj).
    HBM bytes: every weight read once per step, GDN states read + written, each slot's KV cache read
    up to its position."""
    hd = importlib.import_module(PKG + ".hybrid_decode")
    cb = importlib.import_module(PKG + ".cb_engine")
    out = []
    for name, cfg in (("hybrid 64-layer stack (48 GDN + 16 attention, MLPs, LM head)", hd.HybridConfig()),
                      ("48 GDN layers with projections (no attention / MLP / LM head)",
                       hd.HybridConfig(layers=48, full_every=0, mlp=0, vocab=0))):
        g_ = torch.Generator().manual_seed(seed)
        ctx = torch.randint(512, 4097, (N_SLOTS,), generator=g_)
        model = hd.HybridDecoder(cfg, N_SLOTS, ctx, steps + warmup + 2, dev, seed=seed)
        inp = torch.randn(N_SLOTS, cfg.hidden, generator=g_).to(torch.bfloat16).to(dev)
        graph = hd.HybridDecodeGraph(model, inp)
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        packed = [v for L in model.layers for v in vars(L).values() if isinstance(v, cb.PackedWeight)]
        packed += [model.lm_head_p] if model.lm_head_p is not None else []
        wbytes = sum(p.N * p.K * 2 for p in packed)                     # the weights' own bytes
        wbytes += sum(L.conv_w.numel() * 2 for L in model.layers if not L.full)
        sbytes = sum(2 * (model.slots.conv[i].numel() * 2 + model.slots.rec[i].numel() * 4) for i in model.slots.rec)
        # the attention reads each slot's K and V at positions 0..pos: the graph's eager warm-up step
        # and the warmup replays advanced pos to ctx + 1 + warmup before the timed steps
        n_attn = sum(1 for L in model.layers if L.full)
        mean_len = float(ctx.double().mean()) + 2 + warmup + (steps - 1) / 2
        kvbytes = int(n_attn * N_SLOTS * mean_len * cfg.kv_heads * cfg.attn_head * 2 * 2)
        total = wbytes + sbytes + kvbytes
        n_gdn = len(model.slots.rec)
        out.append({"workload": f"decode step, Qwen3.5-27B shape, {name}, 16 slots, ctx U[512,4096], HIP graph",
                    "ms_per_step": round(ms, 3), "tokens_per_s": round(N_SLOTS / ms * 1e3, 1),
                    "us_per_gdn_layer": round(ms * 1e3 / n_gdn, 2) if not cfg.full_every else None,
                    "hbm_bytes_per_step": total, "weight_bytes": wbytes, "gdn_state_bytes": sbytes,
                    "kv_cache_bytes_read": kvbytes,
                    "hbm_frac": round(total / (ms * 1e-3) / HBM_PEAK, 4)})
        del graph, model, inp
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--only", choices=["decode", "prefill", "prefill8192", "varlen", "hybrid", "attention"],
                    default=None, help="run one workload group (prefill8192: the T=8192 chunked rule alone; varlen: "
                                       "the 16-prompt prefill layer alone; both for profiling)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run a 256 MiB device-to-device copy (counter calibration for rocprof)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the GDN path is benchmarked on a single "
              "MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    gdn = importlib.import_module(PKG)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.calib_copy:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)   # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    res = {}
    if args.only in (None, "decode"):
        res["decode"] = bench_decode(gdn, dev, args.steps, args.warmup)
        res["decode_share"] = [bench_decode_tp_share(gdn, dev, args.steps, args.warmup)]
    if args.only == "prefill8192":
        res["prefill"] = [bench_prefill(gdn, dev, reps=args.steps)]
    elif args.only == "varlen":
        res["prefill"] = [bench_prefill_varlen(gdn, dev, reps=args.steps)]
    elif args.only in (None, "prefill") and not args.no_prefill:
        res["prefill"] = [bench_prefill(gdn, dev), bench_prefill_varlen(gdn, dev, cpu=not args.no_cpu),
                          bench_prefill_long(gdn, dev, check=not args.no_cpu),
                          bench_prefill(gdn, dev, T=8192, hv=48),
                          bench_prefill(gdn, dev, T=353, hv=48, reps=20,
                                        note="Qwen3.5-27B's GDN shape at the reference's only published prefill "
                                             "size (its chunk function: 5.64 ms/layer at 353 tokens on its own "
                                             "accelerator, quoted as context only)"),
                          bench_prefill(gdn, dev, T=8192, decay=0.001,
                                        note="slow decay: no segment boundary has a warm-up below 2^-16, so the "
                                             "exact path runs (both summaries of every segment, their fp32 "
                                             "combination, then the outputs), and every chunk decays by less "
                                             "than e^-2 and takes W S in bf16 hi + lo")]
        if not args.no_cpu:
            res["prefill"][0]["cpu_baseline"] = cpu_baseline_prefill()
    if args.only in (None, "hybrid"):
        res["hybrid"] = bench_hybrid(gdn, dev)
    if args.only in (None, "attention"):
        res["hybrid"] = res.get("hybrid", []) + [bench_attention(gdn, dev, reps=args.steps if args.only else 3)]
    if args.only in ("prefill", "prefill8192", "varlen", "hybrid", "attention"):
        print(json.dumps({"secondary": res.get("prefill", []) + res.get("hybrid", [])}))
        return
    dec = res["decode"]
    bpl = decode_bytes_per_layer()
    achieved = bpl / (dec["us_per_layer"] * 1e-6) / 1e9
    line = {
        "metric": "GDN prefill tokens/s/layer (MFMA %); 16-slot decode µs/layer (HBM GB/s %)",
        "value": round(dec["us_per_layer"], 3),
        "unit": "us/layer (16-slot GDN decode step, fused conv+gating+recurrent+gated norm)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 state / bf16 activations", "data": "synthetic (seeded), random-init parameters",
        "config": {"workload": "GDN decode step, 16 slots x 1 token, H_k=16, H_v=32, d=128, conv 8192x4, "
                               "48 distinct layers, HIP-graph replay", "slots": N_SLOTS, "layers": LAYERS},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved * 1e9 / HBM_PEAK, 4), "traffic": DECODE_TRAFFIC,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, copy-calibrated "
                                       "(profiles/decode_fused_kernel_16slot_Hv32_48layer.md)",
                     "kernel": "decode_fused_kernel<2,true>", "algorithmic_bytes_per_launch": bpl,
                     "us_per_launch_graph": round(dec["us_per_layer"], 3),
                     "us_per_launch_eager": round(dec["us_per_layer_eager"], 3)},
    }
    line["secondary"] = res.get("decode_share", []) + res.get("prefill", []) + res.get("hybrid", [])
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_decode()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
