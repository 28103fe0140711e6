"""CPU checks of the host API: the reference-named functions validate their inputs and refuse CPU
tensors (there is no CPU fallback) before any GPU call."""
import pytest
import torch


def test_public_names(gdn):
    for name in ("fast_chunk_gated_delta_rule", "fast_chunk_gated_delta_rule_v2", "recurrent_single_step",
                 "elem_conv_update", "patch_model", "gated_rmsnorm", "gdn_decode_core", "gdn_prefill_core",
                 "causal_conv1d_prefill", "causal_conv1d_update", "GDNSlots", "GDNDecodeGraph"):
        assert hasattr(gdn, name)


def test_cpu_tensors_are_refused(gdn):
    q = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    g = torch.zeros(1, 4, 2)
    with pytest.raises(ValueError, match="no CPU fallback"):
        gdn.fast_chunk_gated_delta_rule_v2(q, q, q, g, g)
    with pytest.raises(ValueError, match="no CPU fallback"):
        gdn.recurrent_single_step(q[:, :1], q[:, :1], q[:, :1], g[:, :1], g[:, :1], None, True)
    x = torch.zeros(2, 16, 1, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no CPU fallback"):
        gdn.elem_conv_update(x, torch.zeros(2, 16, 4, dtype=torch.bfloat16),
                             torch.zeros(16, 4, dtype=torch.bfloat16), None)


def test_cu_seqlens_validation(gdn):
    from importlib import import_module
    cf = import_module(gdn.__name__ + ".gdn_chunk_fast")
    cu, s0, nseq, _, total = cf._chunk_table(1, 200, torch.tensor([0, 64, 64, 130, 200]), "cpu")
    assert nseq == 4 and total == 1 + 0 + 2 + 2 and s0.tolist() == [0, 1, 1, 3, 5]
    for bad in ([0, 50, 40, 200], [1, 200], [0, 100], [0]):
        with pytest.raises(ValueError):
            cf._chunk_table(1, 200, torch.tensor(bad), "cpu")
    with pytest.raises(ValueError):
        cf._chunk_table(2, 100, torch.tensor([0, 100]), "cpu")
    # host lists, tuples and tensors give the same tables (lists skip the tensor round trip)
    for form in ([0, 64, 64, 130, 200], (0, 64, 64, 130, 200), torch.tensor([0, 64, 64, 130, 200], dtype=torch.int32)):
        vl = cf.Varlen(form, 200, "cpu")
        assert vl.cu.tolist() == [0, 64, 64, 130, 200] and vl.seq_chunk0.tolist() == [0, 1, 1, 3, 5]
        assert vl.cu.dtype == vl.seq_chunk0.dtype == torch.int32
        assert (vl.nseq, vl.total_chunks, vl.max_len) == (4, 5, 70)
    for bad in ([0, 50, 40, 200], (1, 200), [0, 100]):
        with pytest.raises(ValueError):
            cf.Varlen(bad, 200, "cpu")
    # slot rows: one per sequence, inside [0, n_rows)
    assert cf.Rows([3, 0, 2], 3, 4, "cpu").dev.tolist() == [3, 0, 2]
    assert cf.Rows(torch.tensor([3, 0, 2]), 3, 4, "cpu").dev.tolist() == [3, 0, 2]
    for rows in ([3, 0], [3, 0, 4], [-1, 0, 2]):
        with pytest.raises(ValueError):
            cf.Rows(rows, 3, 4, "cpu")


def test_patch_model_installs_functions(gdn):
    from transformers.models.qwen3_5 import modeling_qwen3_5 as M
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    saved = (M.torch_chunk_gated_delta_rule, M.torch_recurrent_gated_delta_rule, M.causal_conv1d_update)
    try:
        cfg = Qwen3_5TextConfig(hidden_size=64, linear_num_key_heads=1, linear_num_value_heads=2,
                                linear_key_head_dim=128, linear_value_head_dim=128, num_hidden_layers=1,
                                layer_types=["linear_attention"], intermediate_size=64, num_attention_heads=2,
                                num_key_value_heads=1, head_dim=64, vocab_size=32)
        layer = M.Qwen3_5GatedDeltaNet(cfg, 0)
        norm16 = M.Qwen3_5RMSNorm(64).to(torch.bfloat16)
        norm32 = M.Qwen3_5RMSNorm(64)
        holder = torch.nn.ModuleList([layer, norm16, norm32])
        gdn.patch_model(holder, fast_gdn=True, gdn_v2=True)
        assert layer.chunk_gated_delta_rule is gdn.fast_chunk_gated_delta_rule_v2
        assert layer.recurrent_gated_delta_rule is gdn.recurrent_single_step
        assert M.torch_chunk_gated_delta_rule is gdn.fast_chunk_gated_delta_rule_v2
        assert layer.norm.forward.__func__ is gdn.fused_gated_rmsnorm
        # bf16 Qwen3_5RMSNorm modules get the fused norm (src/cb_engine.py:62-63,70-71); others stay HF's
        assert norm16.forward.__func__ is gdn.fused_rmsnorm
        assert not hasattr(norm32.forward, "__func__") or norm32.forward.__func__ is not gdn.fused_rmsnorm
    finally:
        M.torch_chunk_gated_delta_rule, M.torch_recurrent_gated_delta_rule, M.causal_conv1d_update = saved


def test_decode_step_ops_refuse_cpu_tensors(gdn):
    """The decode-step ops around the core (attention, residual add + norm) have no CPU path either."""
    from importlib import import_module
    from conftest import PKG_NAME
    cb = import_module(PKG_NAME + ".cb_engine")
    N, nh, kv, hd, T = 2, 4, 2, 64, 8
    bf = torch.bfloat16
    proj = torch.zeros(N, (2 * nh + 2 * kv) * hd, dtype=bf)
    with pytest.raises(ValueError, match="no CPU fallback"):
        cb.gqa_decode_attention(proj, torch.zeros(N, dtype=torch.int64), torch.zeros(hd, dtype=bf),
                                torch.zeros(hd, dtype=bf), torch.ones(hd // 8), torch.zeros(N, kv, hd, T, dtype=bf),
                                torch.zeros(N, kv, T, hd, dtype=bf), nh, kv, hd, hd // 4)
    h = torch.zeros(N, 256, dtype=bf)
    with pytest.raises(ValueError, match="no CPU fallback"):
        cb.add_rms_norm(h, h, torch.zeros(256, dtype=bf))


def test_chunk_rule_argument_domain(gdn):
    """The reference's v2 takes any float dtype, head dims and chunk size (src/gdn_chunk_fast2.py:11-29):
    fp32 / bf16 / fp16 q/k/v with d_k, d_v in {16, 32, 64, 128} and any positive chunk_size pass the
    argument checks and reach the device check (CPU tensors: no CPU fallback); mixed or other dtypes,
    other head dims and a chunk size below 1 raise a ValueError naming the domain, before any device work."""
    bf = torch.bfloat16
    q = torch.zeros(1, 4, 2, 128, dtype=bf)
    g = torch.zeros(1, 4, 2)
    for fn in (gdn.fast_chunk_gated_delta_rule, gdn.fast_chunk_gated_delta_rule_v2):
        for x, cs in ((q, 128), (q.float(), 64), (q.half(), 16), (torch.zeros(1, 4, 2, 64), 64)):
            with pytest.raises(ValueError, match="no CPU fallback"):
                fn(x, x, x, g, g, chunk_size=cs)
        with pytest.raises(ValueError, match="chunk_size must be a positive integer"):
            fn(q, q, q, g, g, chunk_size=0)
        qf = q.float()
        with pytest.raises(ValueError, match="dtypes .* are not supported"):
            fn(q, q, qf, g, g)
        with pytest.raises(ValueError, match="dtypes .* are not supported"):
            fn(q.double(), q.double(), q.double(), g, g)
        q96 = torch.zeros(1, 4, 2, 96, dtype=bf)
        with pytest.raises(ValueError, match="head dims 96"):
            fn(q96, q96, q96, g, g)
