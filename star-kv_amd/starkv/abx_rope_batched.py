"""Drop-in for ``abx_rope_batched.abx`` on libstarkv.

``abx(a, b, x, dtype)`` keeps the reference's signature and output contract
(abx_rope_batched.py:135-186): unscaled decode logits
``out[b, q, 0, s] = a[b, q, 0] . RoPE_s(x[b, q // gs, s] @ b[q // gs])`` of
shape ``[B, Hq, 1, S]`` in ``x``'s dtype, position s rotated by its own angle
(the Triton kernel's semantics, abx_rope_batched.py:117-125), ``b`` indexed per
KV head (abx_rope_batched.py:81).  The work runs in the K-logit kernel of the
C ABI (``starkv_k_logits``); argument errors raise ``StarKVError`` instead of
the reference's bare asserts (147-149) and its ``UnboundLocalError`` on an
unsupported ``dtype`` (163-168).
"""
from __future__ import annotations

from typing import Optional

import torch

from ._lib import StarKVError
from .ops import KLatentSpec, k_logits
from .rope import RopeConfig

__all__ = ["abx"]


def abx(a: torch.Tensor, b: torch.Tensor, x: torch.Tensor, dtype: torch.dtype = torch.float16,
        rope: Optional[RopeConfig] = None) -> torch.Tensor:
    """Decode logits A @ RoPE(X @ B)^T without the 1/sqrt(D) scale.

    a: rotated query [B, Hq, 1, 128]; b: ``k_u^T`` [Hkv, r, 128], or with
    more rows -- the reference's own check passes one per query head,
    [Hq, r, 128] (abx_rope_batched.py:254-265) -- of which, as in the Triton
    kernel (row q // gs, abx_rope_batched.py:81), only the first Hkv are read;
    x: key latent cache [B, Hkv, S, r] (last dim contiguous).  ``dtype`` is the
    reference's compute-dtype switch (float16 / bfloat16 / float32); the
    kernel computes in the operands' own dtype with fp32 accumulation, so it
    only selects which inputs are accepted.  ``rope`` (an extension) selects
    theta / llama3 scaling; the reference fixes theta = 10000
    (abx_rope_batched.py:184), which is the default here.
    """
    if a.dim() != 4 or b.dim() != 3 or x.dim() != 4:
        raise StarKVError("abx expects a [B, Hq, 1, D], b [Hkv, r, D], x [B, Hkv, S, r]")
    if dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise StarKVError(f"abx: unsupported dtype {dtype}")
    B, Hq, one, D = a.shape
    if one != 1:
        raise StarKVError("abx is the decode operator: a must hold one query position")
    if x.shape[0] != B or Hq % x.shape[1]:
        raise StarKVError(f"abx: a {tuple(a.shape)} and x {tuple(x.shape)} disagree on batch or heads")
    if not (a.dtype == b.dtype == x.dtype):
        raise StarKVError(f"abx: a, b and x must share one dtype (got {a.dtype}, {b.dtype}, {x.dtype})")
    if b.shape[0] < x.shape[1]:
        raise StarKVError(f"abx: b {tuple(b.shape)} holds fewer than the {x.shape[1]} KV heads of x")
    spec = KLatentSpec.from_reference(x, b[:x.shape[1]])
    out = k_logits(a, spec, seq_len=x.shape[2], rope=rope or RopeConfig(), scale=1.0, out_dtype=x.dtype)
    return out.unsqueeze(2)
