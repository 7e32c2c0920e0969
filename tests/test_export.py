"""CPU tests of the trained-weight export (starkv.export), the counterpart of
the reference's export_kproj_for_triton / export_vproj_for_triton
(model.py:286-362).

The expected projections come from how the factors were built, not from the
export's formula: with alpha = 0 the fold must give back the decomposed
matrix (SVD identity); with orthonormal factors and chosen singular values
the kept product is U_keep diag(sigma - alpha) V_keep."""
import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "star-kv_amd"))

from starkv.export import export_state_dict, fold_global, fold_headwise  # noqa: E402

D = 128


def _orthonormal(n, k, g):
    q, _ = torch.linalg.qr(torch.randn(n, k, generator=g, dtype=torch.float64))
    return q[:, :k]


def _headwise(g, H, hidden, sigmas):
    """Block-diagonal U [H*D, sum r], V [sum r, hidden] with orthonormal blocks."""
    r = [len(s) for s in sigmas]
    U = torch.zeros(H * D, sum(r), dtype=torch.float64)
    V = torch.zeros(sum(r), hidden, dtype=torch.float64)
    off = 0
    for h in range(H):
        U[h * D:(h + 1) * D, off:off + r[h]] = _orthonormal(D, r[h], g)
        V[off:off + r[h]] = _orthonormal(hidden, r[h], g).t()
        off += r[h]
    return U, V


def _k_product(ranks, k_vs, bk):
    """The exported per-head projections B_k^T VS as one [H*D, hidden] matrix."""
    rows, off = [], 0
    for h, r in enumerate(ranks):
        rows.append(bk[h, :r].double().t() @ k_vs[off:off + r].double())
        off += r
    return torch.cat(rows, 0)


def test_alpha_zero_gives_back_the_decomposed_matrices():
    g = torch.Generator().manual_seed(0)
    H, hidden = 4, 256
    Wk = torch.randn(H * D, hidden, generator=g, dtype=torch.float64)
    Wv = torch.randn(H * D, hidden, generator=g, dtype=torch.float64)
    # per-head SVD of k_proj (model.py:136-174) and one SVD of v_proj (model.py:195-198)
    Us, Ss, Vs = zip(*[torch.linalg.svd(Wk[h * D:(h + 1) * D], full_matrices=False) for h in range(H)])
    U = torch.block_diag(*Us)
    V = torch.cat(Vs, 0)
    ranks, k_vs, bk = fold_headwise(U, V, list(Ss), [0.0] * H, dtype=torch.float64)
    assert ranks == [D] * H
    assert torch.allclose(_k_product(ranks, k_vs, bk), Wk, atol=1e-10)
    Uv, Sv, Vv = torch.linalg.svd(Wv, full_matrices=False)
    v_vs, v_u = fold_global(Uv, Vv, Sv, 0.0, dtype=torch.float64)
    assert v_vs.shape[0] == Sv.numel()
    assert torch.allclose(v_u @ v_vs, Wv, atol=1e-10)


def test_thresholds_keep_and_shift_the_singular_values():
    g = torch.Generator().manual_seed(1)
    H, hidden = 3, 192
    sigmas = [torch.tensor([5.0, 0.3, 2.0, 0.9, 1.5]), torch.tensor([0.2, 4.0, 0.1]),
              torch.tensor([3.0, 2.5, 2.0, 1.0, 0.5, 0.25])]
    alphas = [1.0, 0.15, 0.75]
    U, V = _headwise(g, H, hidden, sigmas)
    ranks, k_vs, bk = fold_headwise(U, V, sigmas, alphas, pad_multiple=1, dtype=torch.float64)
    assert ranks == [3, 2, 4]
    expect, off = [], 0
    for h in range(H):
        s = sigmas[h].double()
        keep = s > alphas[h]
        Uh = U[h * D:(h + 1) * D, off:off + len(s)][:, keep]
        Vh = V[off:off + len(s)][keep]
        expect.append(Uh @ torch.diag(s[keep] - alphas[h]) @ Vh)
        off += len(s)
    assert torch.allclose(_k_product(ranks, k_vs, bk), torch.cat(expect, 0), atol=1e-12)
    # padding with zero rows to a multiple of 8 changes nothing
    ranks8, k_vs8, bk8 = fold_headwise(U, V, sigmas, alphas, pad_multiple=8, dtype=torch.float64)
    assert ranks8 == [8, 8, 8]
    assert torch.allclose(_k_product(ranks8, k_vs8, bk8), torch.cat(expect, 0), atol=1e-12)


def test_min_rank_truncation_matches_the_reference_export():
    """ragged=False keeps, per head, the first min(kept) kept ranks in index
    order (model.py:316-318)."""
    g = torch.Generator().manual_seed(2)
    sigmas = [torch.tensor([0.1, 3.0, 2.0, 4.0]), torch.tensor([2.0, 0.1, 1.5, 1.2, 5.0]), torch.tensor([1.0, 2.0])]
    alpha = 0.5
    U, V = _headwise(g, 3, 160, sigmas)
    ranks, k_vs, bk = fold_headwise(U, V, sigmas, [alpha] * 3, ragged=False, pad_multiple=1, dtype=torch.float64)
    assert ranks == [2, 2, 2]
    expect, off = [], 0
    for s in sigmas:
        s = s.double()
        keep = (s > alpha).nonzero().view(-1)[:2]
        h = len(expect)
        Uh = U[h * D:(h + 1) * D, off + keep]
        expect.append(Uh @ torch.diag(s[keep] - alpha) @ V[off + keep])
        off += len(s)
    assert torch.allclose(_k_product(ranks, k_vs, bk), torch.cat(expect, 0), atol=1e-12)


def test_a_head_that_keeps_nothing_keeps_one_zero_rank():
    g = torch.Generator().manual_seed(3)
    sigmas = [torch.tensor([0.2, 0.1]), torch.tensor([3.0, 1.0])]
    U, V = _headwise(g, 2, 128, sigmas)
    ranks, k_vs, bk = fold_headwise(U, V, sigmas, [0.5, 0.5], pad_multiple=1, dtype=torch.float64)
    assert ranks == [1, 2]
    assert torch.count_nonzero(k_vs[0]) == 0
    v_vs, v_u = fold_global(U[:D, :2], V[:2], sigmas[0], 0.5, pad_multiple=1, dtype=torch.float64)
    assert v_vs.shape[0] == 1 and torch.count_nonzero(v_u @ v_vs) == 0


def test_state_dict_with_the_reference_keys():
    g = torch.Generator().manual_seed(4)
    H, hidden = 2, 128
    sigmas = [torch.linspace(3.0, 0.1, D), torch.linspace(2.0, 0.05, D)]
    U, V = _headwise(g, H, hidden, sigmas)
    Uv = _orthonormal(H * D, 96, g)
    Vv = _orthonormal(hidden, 96, g).t()
    sv = torch.linspace(4.0, 0.01, 96)
    sd = {"k_proj.U.weight": U.float(), "k_proj.V.weight": V.float(),
          "v_proj.U.weight": Uv.float(), "v_proj.V.weight": Vv.float(),
          "v_proj.Sigma.diag": sv, "v_proj.Sigma.soft_thres_layer.alpha": torch.tensor([0.5])}
    for h in range(H):
        sd[f"k_proj.Sigma_blocks.{h}.diag"] = sigmas[h]
        sd[f"k_proj.Sigma_blocks.{h}.soft_thres_layer.alpha"] = torch.tensor([0.4 + 0.2 * h])
    p = export_state_dict(sd, dtype=torch.float32)
    alphas = [float(sd[f"k_proj.Sigma_blocks.{h}.soft_thres_layer.alpha"]) for h in range(H)]   # fp32 values
    ranks, k_vs, bk = fold_headwise(U.float(), V.float(), sigmas, alphas, dtype=torch.float32)
    assert p.ranks == ranks and all(r % 8 == 0 for r in p.ranks)
    assert torch.equal(p.k_vs, k_vs) and torch.equal(p.bk, bk)
    v_vs, v_u = fold_global(Uv.float(), Vv.float(), sv, 0.5, dtype=torch.float32)
    assert torch.equal(p.v_vs, v_vs) and torch.equal(p.v_u, v_u)
    assert p.v_vs.shape[0] % 8 == 0


def test_layout_errors():
    with pytest.raises(ValueError):
        fold_headwise(torch.zeros(2 * D, 10), torch.zeros(10, 64), [torch.ones(4), torch.ones(4)], [0.0, 0.0])
    with pytest.raises(ValueError):
        fold_global(torch.zeros(D, 4), torch.zeros(5, 64), torch.ones(4), 0.0)
