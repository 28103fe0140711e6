"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the oracle and
cross-checked against transformers there): the oracle must keep reproducing them on the CPU, and the
HIP kernels must match them on the GPU within the path's tolerances."""
import os

import numpy as np
import pytest
import torch

from conftest import ROOT, rel_l2

GOLD = os.path.join(ROOT, "tests", "golden")
PREFILL_T = [1, 63, 64, 65, 130]


def load(name):
    with np.load(os.path.join(GOLD, name), allow_pickle=False) as f:
        out = {}
        for k in f.files:
            a = f[k]
            out[k] = torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16) if a.dtype == np.uint16 \
                else torch.from_numpy(a)
        return out


@pytest.mark.parametrize("T", PREFILL_T)
def test_oracle_reproduces_prefill_fixture(oracle, T):
    d = load(f"prefill_T{T}.npz")
    o, s = oracle.chunk_gated_delta_rule_v2(d["q"], d["k"], d["v"], d["g"], d["beta"], 64, d["s0"], True, True)
    assert rel_l2(o, d["out"]) <= 1e-3 and rel_l2(s, d["state"]) <= 1e-6


def test_oracle_reproduces_decode_and_conv_fixtures(oracle):
    d = load("decode_N2.npz")
    conv, rec = d["conv_state"].clone(), d["rec_state"].clone()
    out = oracle.gdn_decode_core(d["mixed"], d["z"], d["a"], d["b"], conv, d["conv_weight"], d["A_log"],
                                 d["dt_bias"], d["norm_weight"], rec, 1, 1, 128)
    assert torch.equal(conv, d["conv_out"])
    assert rel_l2(out, d["out"]) <= 1e-3 and rel_l2(rec, d["rec_out"]) <= 1e-6
    c = load("conv_kat.npz")
    st = c["state"].clone()
    o = oracle.elem_conv_update(c["x"], st, c["w"], None)
    assert torch.equal(o, c["out"]) and torch.equal(st, c["state_out"])


@pytest.mark.gpu
@pytest.mark.parametrize("T", PREFILL_T)
def test_hip_prefill_matches_fixture(gdn, dev, T):
    d = {k: v.to(dev) for k, v in load(f"prefill_T{T}.npz").items()}
    o, s = gdn.fast_chunk_gated_delta_rule_v2(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["s0"],
                                              output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_l2(o, d["out"]) <= 1e-2 and rel_l2(s, d["state"]) <= 1e-3


@pytest.mark.gpu
def test_hip_decode_and_conv_match_fixtures(gdn, dev):
    d = {k: v.to(dev) for k, v in load("decode_N2.npz").items()}
    out = gdn.gdn_decode_core(d["mixed"], d["z"], d["a"], d["b"], d["conv_state"], d["conv_weight"], d["A_log"],
                              d["dt_bias"], d["norm_weight"], d["rec_state"], 1, 1, 128)
    assert torch.equal(d["conv_state"].cpu(), d["conv_out"].cpu())
    assert rel_l2(out, d["out"]) <= 1e-2 and rel_l2(d["rec_state"], d["rec_out"]) <= 1e-3
    c = {k: v.to(dev) for k, v in load("conv_kat.npz").items()}
    o = gdn.elem_conv_update(c["x"], c["state"], c["w"], None)
    assert torch.equal(o.cpu(), c["out"].cpu()) and torch.equal(c["state"].cpu(), c["state_out"].cpu())
