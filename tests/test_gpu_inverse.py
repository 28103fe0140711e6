"""GPU parity of the chunked prefill's intra-chunk inverse (src/gdn_chunk_fast.py:21-62,
src/gdn_chunk_fast2.py:39-43) -- the routine the hot path runs, checked on its own.

* gdn_unit_lower_inv runs reg_inv64, the register inverse of the prefill's inverse kernel: against
  torch.linalg.solve_triangular (fp64) and the oracle's blocked inverse at 1e-5 rel-L2, T (I - X) = I.
* gdn_chunk_prefill_inverse runs the inverse kernel itself (inv_kernel) and expands the T diag(beta)
  records it hands to the output pass: against the oracle's (I - X)^-1 diag(beta) built from the
  reference's own bf16 l2-normalised keys.  The kernel forms K K^T from those same rounded rows and
  stores bf16 values, so its records are the oracle's rounded to bf16 up to the fp32 order of the
  two inverses: within 5e-4 rel-L2 of bf16(oracle) (a few one-ulp flips).  Against the oracle's fp32
  values the bf16 store alone is 1e-4 to 3e-4 rel-L2 with bf16 beta and up to 1.6e-3 overall / 2.9e-3
  per matrix with fp32 beta (a diagonal of non-bf16 values), so that bound is 2e-3 / 3e-3.  Exact
  zeros where the algebra puts them: above the diagonal, the rows and columns of beta = 0 tokens, the
  rows past a chunk's end.  The K rows' l2norm factors are checked through
  bf16(k * factor) == the reference's normalised rows, bit for bit on all rows but at most one (the
  kernel's fp32 sum order flips the bf16 rounding of the sum of squares for ~5 rows in a million).
"""
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _x_matrices(n, seed, decay=0.1, zero_beta_rows=(), positive_g=False):
    g_ = torch.Generator().manual_seed(seed)
    k = torch.nn.functional.normalize(torch.randn(n, 64, 128, generator=g_), dim=-1)
    beta = torch.rand(n, 64, generator=g_)
    for i in zero_beta_rows:
        beta[:, i] = 0.0
    gg = torch.rand(n, 64, generator=g_) * decay
    G = torch.cumsum(gg if positive_g else -gg, dim=-1)
    dec = (G.unsqueeze(-1) - G.unsqueeze(-2)).tril().exp().tril()
    return -((k * beta.unsqueeze(-1)) @ k.transpose(-1, -2) * dec).tril(-1)


@pytest.mark.parametrize("case,seed", [("decay", 1), ("slow", 2), ("zero_beta_rows", 3), ("positive_g", 4),
                                       ("odd_batch", 5)])
def test_unit_lower_inv_is_the_register_inverse(gdn, oracle, dev, case, seed):
    n = 37 if case == "odd_batch" else 64   # 37: the last workgroup has one live wave
    X = _x_matrices(n, seed=seed,
                    decay={"slow": 0.005, "positive_g": 0.02}.get(case, 0.3),
                    zero_beta_rows=(0, 5, 17, 63) if case == "zero_beta_rows" else (),
                    positive_g=case == "positive_g")
    Xd = X + torch.triu(torch.full_like(X, 7.0), 0)  # entries on and above the diagonal are not read
    T = gdn._unit_lower_inv(Xd.to(dev)).cpu()
    I = torch.eye(64)
    exact = torch.linalg.solve_triangular((I - X).double(), I.double().expand(n, 64, 64), upper=False)
    assert rel_l2(T, exact) <= 1e-5, rel_l2(T, exact)
    assert rel_l2(T, oracle.unit_lower_inv(X)) <= 1e-5
    assert ((T.double() @ (I - X).double()) - I.double()).abs().max().item() <= 1e-4
    assert torch.equal(torch.triu(T, 1), torch.zeros_like(T)), "upper triangle must be exactly zero"
    assert torch.equal(torch.diagonal(T, dim1=-2, dim2=-1), torch.ones(n, 64))


def _oracle_records(oracle, k, g, beta, lens, Hv):
    """Per chunk and value head: (I - X)^-1 diag(beta), X from the reference's bf16 l2-normalised keys
    (src/gdn_chunk_fast2.py:14-16, :31-43), sequences padded to whole chunks with zeros."""
    r = Hv // k.shape[1]
    out, t0 = [], 0
    kn_all = oracle.l2norm(k).float()
    for L in lens:
        n = (L + 63) // 64
        kn = torch.zeros(n * 64, k.shape[1], 128)
        kn[:L] = kn_all[t0:t0 + L]
        gp = torch.zeros(n * 64, Hv)
        gp[:L] = g[t0:t0 + L]
        bp = torch.zeros(n * 64, Hv)
        bp[:L] = beta[t0:t0 + L].float()
        kc = kn.reshape(n, 64, -1, 128).repeat_interleave(r, dim=2).permute(0, 2, 1, 3)  # [n, Hv, 64, 128]
        G = gp.reshape(n, 64, Hv).permute(0, 2, 1).cumsum(-1)
        b = bp.reshape(n, 64, Hv).permute(0, 2, 1)
        dec = (G.unsqueeze(-1) - G.unsqueeze(-2)).tril().exp().tril()
        X = -((kc * b.unsqueeze(-1)) @ kc.transpose(-1, -2) * dec).tril(-1)
        out.append(oracle.unit_lower_inv(X) * b.unsqueeze(-2))
        t0 += L
    return torch.cat(out, dim=0)


@pytest.mark.parametrize("lens,Hk,Hv,decay,beta_dtype", [
    ([1], 1, 2, 0.1, torch.bfloat16),                # one token: a 1x1 inverse in a padded chunk
    ([63], 2, 2, 0.1, torch.bfloat16),               # one short chunk
    ([65], 2, 4, 0.1, torch.float32),                # a full chunk and a 1-token tail; fp32 beta
    ([130, 64, 1, 257], 2, 4, 0.005, torch.bfloat16),  # packed sequences, slow decay
    ([300], 4, 12, 0.1, torch.bfloat16),             # ratio 3
])
def test_inverse_kernel_records_match_the_oracle(gdn, oracle, dev, lens, Hk, Hv, decay, beta_dtype):
    T = sum(lens)
    g_ = torch.Generator().manual_seed(T + Hv)
    k = torch.randn(T, Hk, 128, generator=g_).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(T, Hv, generator=g_))
    beta[::7] = 0.0                                 # beta = 0 tokens (every 7th)
    beta = beta.to(beta_dtype)
    g = -torch.nn.functional.softplus(torch.randn(T, Hv, generator=g_) + 2) * decay
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    Td, fac = gdn.chunk_inverse_records(k.unsqueeze(0).to(dev), g.unsqueeze(0).to(dev), beta.unsqueeze(0).to(dev),
                                        cu_seqlens=cu if len(lens) > 1 else None)
    Td, fac = Td.cpu(), fac.cpu()
    ref = _oracle_records(oracle, k, g, beta, lens, Hv)
    assert Td.shape == ref.shape
    ref_bf = ref.to(torch.bfloat16).float()
    assert rel_l2(Td, ref_bf) <= 5e-4, rel_l2(Td, ref_bf)
    assert rel_l2(Td, ref) <= 2e-3, rel_l2(Td, ref)
    per = ((Td - ref).flatten(2).norm(dim=-1) / ref.flatten(2).norm(dim=-1).clamp_min(1e-30)).max().item()
    assert per <= 3e-3, per
    # exact zeros: upper triangle, beta = 0 columns and rows, rows and columns past each chunk's end
    assert torch.equal(torch.triu(Td, 1), torch.zeros_like(Td))
    zero = ref == 0
    assert torch.equal(Td[zero], torch.zeros_like(Td[zero])), "the kernel put values where the algebra has none"
    # the l2norm factors: bf16(k * factor) is the reference's normalised key row, bit for bit.  The
    # kernel sums the bf16 squares in another fp32 order than torch; that moves the bf16 sum by one
    # ulp for about 5 rows in a million (measured on the CPU), so one row may differ
    r = Hv // Hk
    t0, c0, rows_seen, rows_off = 0, 0, 0, 0
    kn = oracle.l2norm(k)
    for L in lens:
        n = (L + 63) // 64
        for c in range(n):
            m = min(64, L - 64 * c)
            for h in (0, Hv - 1):
                f = fac[c0 + c, h, :m]
                got = (k[t0 + 64 * c:t0 + 64 * c + m, h // r].float() * f.unsqueeze(-1)).to(torch.bfloat16)
                want = kn[t0 + 64 * c:t0 + 64 * c + m, h // r]
                rows_seen += m
                rows_off += int((got != want).any(dim=-1).sum())
        t0 += L
        c0 += n
    assert rows_off <= 1, f"{rows_off} of {rows_seen} normalised key rows differ from the reference's"
