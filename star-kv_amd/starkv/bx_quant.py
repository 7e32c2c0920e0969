"""Drop-in for ``bx_quant.bx`` on libstarkv.

``bx(b, x1, x2, scale_v_upper, scale_v_lower, original_rank, upper_rank=256)``
keeps the reference's signature (bx_quant.py:117-166) and returns
``out[b, h, j] = sum_s P[b, h, s] * V[b, s, j]`` of shape [B, H, R] in P's
dtype, with V dequantised from the reference's split cache: ranks
[0, upper_rank) from ``x1`` and ranks [upper_rank, R) from ``x2``, each with
one fp16 scale per token, int4 nibbles with value ``(nibble - 8) * s``
(bx_quant.py:75-86).  ``x1`` may also hold int8 values ([B, S, upper_rank]
int8, the reading of LlamaLoRaAttention_headwise_quant.py:138, 164); its last
dimension tells which.

Differences from the reference, on purpose: the output is fully written by a
deterministic split-S reduction (the reference allocates it with
``torch.empty`` and adds fp16 atomics into it, bx_quant.py:113-114, 147), and
any H <= 32 is accepted (the reference hard-codes 32, bx_quant.py:148).
"""
from __future__ import annotations

import torch

from ._lib import StarKVError
from .ops import VLatentSpec, pv_latent

__all__ = ["bx"]


def bx(b: torch.Tensor, x1: torch.Tensor, x2: torch.Tensor, scale_v_upper: torch.Tensor,
       scale_v_lower: torch.Tensor, original_rank: int, upper_rank: int = 256) -> torch.Tensor:
    """P @ dequant(V) for the decode step.

    b: probabilities [B, H, S] (act dtype); x1: upper V cache [B, S, upper_rank/2]
    uint8 (or [B, S, upper_rank] int8); x2: lower V cache [B, S, (R - upper_rank)/2]
    uint8; scale_v_upper / scale_v_lower: fp16 [B, S, 1]; original_rank: R.
    """
    if b.dim() != 3 or x1.dim() != 3:
        raise StarKVError("bx expects b [B, H, S] and x1 [B, S, bytes]")
    R, U = int(original_rank), int(upper_rank)
    if not 0 < U <= R:
        raise StarKVError(f"bx: upper_rank {U} must lie in (0, original_rank {R}]")
    if U < R and (x2 is None or x2.dim() != 3):
        raise StarKVError("bx: x2 must be [B, S, bytes] when original_rank > upper_rank")
    for t, name in ((scale_v_upper, "scale_v_upper"), (scale_v_lower, "scale_v_lower")):
        if t is not None and t.dtype != torch.float16:
            raise StarKVError(f"bx: {name} must be float16 per-token scales")
    spec = VLatentSpec.int4_ref(x1, scale_v_upper, R, split=U,
                                x2=x2 if U < R else None, scale2=scale_v_lower if U < R else None)
    return pv_latent(b, spec)
