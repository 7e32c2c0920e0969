"""Trained-weight export: fold the soft-thresholded singular values into the
latent projections and keep every KV head's own rank.

Mirrors the reference's `export_kproj_for_triton` / `export_vproj_for_triton`
(model.py:286-362), which turn a trained decomposition W ~ U diag(sigma) V
(`DecomposeLinear_headwise` for k_proj, one SVD block per KV head,
model.py:76-174; `DecomposeLinear` for v_proj, model.py:177-205) into the
inference layout:

* keep the ranks whose learned `diag` exceeds the head's threshold alpha
  (model.py:306-309, 344-347; a head that keeps none keeps rank 0 with a zero
  scale);
* fold s = (diag - alpha).clamp_min(0) into the rows of V (model.py:310-312,
  348-350) -- the inference fold, not the training-time soft threshold
  x * tanh(s (x - alpha)) of soft_thres_layer.py:20-26;
* K: VS rows [sum of kept ranks, hidden] and per-head U columns
  (model.py:313-314); V: VS [kept, hidden] and U [out, kept] (model.py:350-351).

The reference then truncates every K head to the layer's smallest kept rank
(model.py:316-318).  `fold_headwise(..., ragged=True)` (the default) keeps the
ragged ranks instead -- the decode kernels take a rank per head -- and
`ragged=False` reproduces the truncation.  Kept ranks can be padded with zero
rows to a multiple (8 by default: quantised caches and the aligned kernels
need it); zero rows add nothing to any product.

Inputs are plain tensors (or a state dict with the reference module's key
names, `export_state_dict`); nothing from the reference is imported.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Mapping, Optional, Sequence

import torch

__all__ = ["LatentProjections", "fold_headwise", "fold_global", "export_state_dict"]


@dataclass
class LatentProjections:
    """One layer's exported latent projections in the layout of
    `starkv.e2e.LatentAttention` / the C ABI:

    ranks   kept K rank per KV head (after padding)
    k_vs    [sum(ranks), hidden]   latent K projection, heads back to back
    bk      [Hkv, max(ranks), 128] B_k = U_h^T per head (rows past r_h zero)
    v_vs    [Rv, hidden]           latent V projection
    v_u     [Hkv*128, Rv]          U_v
    """
    ranks: List[int]
    k_vs: torch.Tensor
    bk: torch.Tensor
    v_vs: torch.Tensor
    v_u: torch.Tensor


def _kept(diag: torch.Tensor, alpha: float):
    """Indices with diag > alpha (index order) and their folded scales
    (model.py:306-310); a head with none keeps index 0 with scale 0."""
    d = diag.detach().double().reshape(-1)
    keep = (d > alpha).nonzero(as_tuple=False).view(-1)
    if keep.numel() == 0:
        keep = torch.zeros(1, dtype=torch.long, device=d.device)
    return keep, (d[keep] - alpha).clamp_min(0)


def _pad(n: int, multiple: int) -> int:
    return n if multiple <= 1 else -(-n // multiple) * multiple


def fold_headwise(U: torch.Tensor, V: torch.Tensor, diags: Sequence[torch.Tensor], alphas: Sequence[float],
                  head_dim: int = 128, ragged: bool = True, pad_multiple: int = 8,
                  dtype: torch.dtype = torch.float16):
    """K projection, one SVD block per KV head (export_kproj_for_triton,
    model.py:287-326).

    U      [Hkv*head_dim, r_total]  the decomposition's U weight (block diagonal by head)
    V      [r_total, hidden]        its V weight
    diags  per head, the learned singular values (length r_h each; their
           lengths give the per-head column ranges of U and V, model.py:302-315)
    alphas per head, the soft-threshold alpha

    Returns (ranks, k_vs [sum(ranks), hidden], bk [Hkv, max(ranks), head_dim]).
    """
    H = len(diags)
    if len(alphas) != H or U.shape[0] != H * head_dim or U.shape[1] != V.shape[0]:
        raise ValueError("fold_headwise: U, V, diags and alphas disagree on the head layout")
    if sum(int(d.numel()) for d in diags) != V.shape[0]:
        raise ValueError("fold_headwise: the diag lengths must sum to the rank of U and V")
    Uw, Vw = U.detach().double(), V.detach().double()
    vs, us = [], []
    off = 0
    for h in range(H):
        keep, s = _kept(diags[h], float(alphas[h]))
        cols = off + keep.to(Uw.device)
        vs.append(Vw[cols] * s.to(Vw.device)[:, None])                  # [k_h, hidden]
        us.append(Uw[h * head_dim:(h + 1) * head_dim][:, cols])         # [head_dim, k_h]
        off += int(diags[h].numel())
    if not ragged:                                                      # model.py:316-318
        m = min(v.shape[0] for v in vs)
        vs, us = [v[:m] for v in vs], [u[:, :m] for u in us]
    ranks = [_pad(v.shape[0], pad_multiple) for v in vs]
    if max(ranks) > head_dim:
        raise ValueError("fold_headwise: a head keeps more ranks than head_dim")
    hidden = Vw.shape[1]
    k_vs = torch.zeros(sum(ranks), hidden, dtype=torch.float64, device=Vw.device)
    bk = torch.zeros(H, max(ranks), head_dim, dtype=torch.float64, device=Uw.device)
    row = 0
    for h in range(H):
        k = vs[h].shape[0]
        k_vs[row:row + k] = vs[h]
        bk[h, :k] = us[h].t()
        row += ranks[h]
    return ranks, k_vs.to(dtype), bk.to(dtype)


def fold_global(U: torch.Tensor, V: torch.Tensor, diag: torch.Tensor, alpha: float, pad_multiple: int = 8,
                dtype: torch.dtype = torch.float16):
    """V projection, one SVD (export_vproj_for_triton, model.py:329-362).

    Returns (v_vs [Rv, hidden], v_u [out, Rv]) with Rv the kept rank padded to
    `pad_multiple` by zero rows / columns."""
    if U.shape[1] != V.shape[0] or int(diag.numel()) != V.shape[0]:
        raise ValueError("fold_global: U, V and diag disagree on the rank")
    Uw, Vw = U.detach().double(), V.detach().double()
    keep, s = _kept(diag, float(alpha))
    keep = keep.to(Vw.device)
    k = int(keep.numel())
    rv = _pad(k, pad_multiple)
    v_vs = torch.zeros(rv, Vw.shape[1], dtype=torch.float64, device=Vw.device)
    v_u = torch.zeros(Uw.shape[0], rv, dtype=torch.float64, device=Uw.device)
    v_vs[:k] = Vw[keep] * s.to(Vw.device)[:, None]
    v_u[:, :k] = Uw[:, keep]
    return v_vs.to(dtype), v_u.to(dtype)


def export_state_dict(sd: Mapping[str, torch.Tensor], k_prefix: str = "k_proj.", v_prefix: str = "v_proj.",
                      head_dim: int = 128, ragged: bool = True, pad_multiple: int = 8,
                      dtype: torch.dtype = torch.float16,
                      n_kv_heads: Optional[int] = None) -> LatentProjections:
    """Export one layer from a state dict with the reference modules' keys
    (model.py:76-205): `{k}U.weight`, `{k}V.weight`,
    `{k}Sigma_blocks.<h>.diag`, `{k}Sigma_blocks.<h>.soft_thres_layer.alpha`,
    `{v}U.weight`, `{v}V.weight`, `{v}Sigma.diag`,
    `{v}Sigma.soft_thres_layer.alpha`.  The U / V weights are used as stored,
    without their masks, as the reference's export does (model.py:297-298,
    340-341)."""
    H = n_kv_heads
    if H is None:
        H = 0
        while f"{k_prefix}Sigma_blocks.{H}.diag" in sd:
            H += 1
    if H == 0:
        raise KeyError(f"no {k_prefix}Sigma_blocks.<h>.diag entries")
    diags = [sd[f"{k_prefix}Sigma_blocks.{h}.diag"] for h in range(H)]
    alphas = [float(sd[f"{k_prefix}Sigma_blocks.{h}.soft_thres_layer.alpha"].reshape(-1)[0]) for h in range(H)]
    ranks, k_vs, bk = fold_headwise(sd[f"{k_prefix}U.weight"], sd[f"{k_prefix}V.weight"], diags, alphas,
                                    head_dim=head_dim, ragged=ragged, pad_multiple=pad_multiple, dtype=dtype)
    v_vs, v_u = fold_global(sd[f"{v_prefix}U.weight"], sd[f"{v_prefix}V.weight"], sd[f"{v_prefix}Sigma.diag"],
                            float(sd[f"{v_prefix}Sigma.soft_thres_layer.alpha"].reshape(-1)[0]),
                            pad_multiple=pad_multiple, dtype=dtype)
    return LatentProjections(ranks, k_vs, bk, v_vs, v_u)
