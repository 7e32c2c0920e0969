"""Drop-in for ``abx_rope_batched_quant.abx`` on libstarkv.

The reference imports ``abx_rope_batched_quant.abx`` without shipping it
(LlamaLoRaAttention_headwise_quant.py:12); its call site fixes the signature,
``abx(A, B, X1, X2, s_k_up, s_k_lo, r4_k)`` (145-152), and the module's
no-kernel branch fixes the semantics (137-144): the key latent is
``cat(X1 * s_k_up, unpack_int4(X2, r4_k) * s_k_lo)`` rounded to the act dtype,
multiplied by ``B`` (k_u^T) and rotated; the result is the unscaled decode
logits [B, Hq, 1, S].  Here keys are rotated by their own positions (the
reference's no-kernel branch uses the last position for all keys,
LlamaLoRaAttention_headwise_quant.py:28-35) and every value is dequantised to
fp16 bit-exactly before use.  The work runs in the K-logit kernel of the C ABI.

``X1``: int8 [B, H, S, u] (the "int8 upper" block; a uint8 tensor of u/2
nibbles per token is read as int4); ``X2``: uint8 int4 nibbles
[B, H, S, r4_k/2] (rank 2k in the low nibble of byte k, value nibble - 8);
``s_k_up`` / ``s_k_lo``: fp16 [B, H, S, 1]; ``H`` = Hkv, or Hq when the caller
repeated the cache per query head as the reference module does (146-147).
"""
from __future__ import annotations

from typing import Optional

import torch

from ._lib import StarKVError
from .ops import KLatentSpec, k_logits
from .rope import RopeConfig

__all__ = ["abx"]


def abx(A: torch.Tensor, B: torch.Tensor, X1: torch.Tensor, X2: torch.Tensor, s_k_up: torch.Tensor,
        s_k_lo: torch.Tensor, r4_k: int, rope: Optional[RopeConfig] = None) -> torch.Tensor:
    """Unscaled decode logits [B, Hq, 1, S] from the split quantised K cache."""
    if A.dim() != 4 or A.shape[2] != 1:
        raise StarKVError("abx expects A [B, Hq, 1, 128] (one decode position)")
    if X1.dim() != 4 or (X2 is not None and X2.dim() != 4):
        raise StarKVError("abx expects X1, X2 [B, H, S, bytes]")
    upper = X1.shape[3] if X1.dtype == torch.int8 else 2 * X1.shape[3]
    rank = upper + int(r4_k)
    if B.dim() != 3 or B.shape[1] != rank:
        raise StarKVError(f"abx: B must be [Hkv, {rank}, 128] (upper {upper} + lower {int(r4_k)} ranks)")
    if A.dtype != B.dtype:
        raise StarKVError("abx: A and B must share the act dtype")
    lower = X2 if int(r4_k) > 0 else None
    spec = KLatentSpec.from_reference_quant(X1, s_k_up, B.contiguous(), rank, x2=lower,
                                            s2=s_k_lo if lower is not None else None, split=upper)
    out = k_logits(A, spec, seq_len=X1.shape[2], rope=rope or RopeConfig(), scale=1.0, out_dtype=A.dtype)
    return out.unsqueeze(2)
