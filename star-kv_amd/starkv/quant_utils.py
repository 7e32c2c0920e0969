"""The reference's missing ``quant_utils`` (imported at bx_quant.py:18 and
LlamaLoRaAttention_headwise_quant.py:14, not shipped).

Its two functions are defined by their call sites:

* ``quantize_r_split_int8_int4_packed(x, split_r)``
  (LlamaLoRaAttention_headwise_quant.py:107-117) returns
  ``(upper_q, scale_upper, lower_q, scale_lower, r4)``: ranks [0, split_r) as
  int8 with one fp16 scale per token ("Top-r ranks stored in int8", 22-25),
  ranks [split_r, R) as packed int4 with one fp16 scale per token
  (ceil(r4 / 2) bytes per token; an odd r4 leaves the last high nibble at 8,
  the value 0), and ``r4 = R - split_r``.  Any R >= split_r is accepted (the
  reference module splits K at 16 and V at 256 ranks; its ``bx`` check runs
  R = 1228, a 972-rank lower block of 486-byte rows, bx_quant.py:224-248).  Build-defined rounding (the reference's is unknown):
  s = fp16(amax / 127) and q = clip(rint(x / s), -127, 127) for int8;
  s = fp16(amax / 7) and n = clip(rint(x / s), -8, 7), stored as nibble n + 8
  with rank 2k in the low nibble of byte k, for int4.  Runs on the HIP cache
  writer (``starkv_k_append`` / ``starkv_v_append``).
* ``unpack_uint8_to_int4_signed(q, r)`` (…_quant.py:139, 165; bx_quant.py:171)
  returns the signed int4 values [..., r] as int8.
"""
from __future__ import annotations

import torch

from ._lib import FMT_INT4_REF, FMT_INT8_SYM, StarKVError
from .ops import KLatentSpec, VLatentSpec, k_append, v_append

__all__ = ["quantize_r_split_int8_int4_packed", "unpack_uint8_to_int4_signed"]


def quantize_r_split_int8_int4_packed(x: torch.Tensor, split_r: int):
    """x: K latent [B, H, T, R] or V latent [B, T, R] (fp16 / bf16, on the GPU)."""
    R, U = x.shape[-1], int(split_r)
    if not 0 < U <= R or U % 16:
        raise StarKVError(f"split_r {U} must be a multiple of 16 in (0, {R}]")
    x = x if x.stride(-1) == 1 else x.contiguous()
    dev = x.device
    lead = x.shape[:-1]
    up = torch.empty(*lead, U, dtype=torch.int8, device=dev)
    lo = torch.empty(*lead, (R - U + 1) // 2, dtype=torch.uint8, device=dev)
    s_up = torch.empty(*lead, 1, dtype=torch.float16, device=dev)
    s_lo = torch.empty(*lead, 1, dtype=torch.float16, device=dev)
    if x.dim() == 4:
        B, H, T, _ = x.shape
        spec = KLatentSpec(up, [R] * H, [h * up.stride(1) for h in range(H)], [up.stride(2)] * H, up.stride(0),
                           x, [0] * H, 128, fmt=FMT_INT4_REF, scale=s_up, scale_stride_b=s_up.stride(0),
                           scale_stride_h=s_up.stride(1), split=U, split_fmt=FMT_INT8_SYM, data2=lo,
                           head_offset2=[h * lo.stride(1) for h in range(H)], pos_stride2=[lo.stride(2)] * H,
                           stride2_b=lo.stride(0), scale2=s_lo, scale2_stride_b=s_lo.stride(0),
                           scale2_stride_h=s_lo.stride(1))
        k_append(x, spec, 0, T)
    elif x.dim() == 3:
        spec = VLatentSpec.int4_ref(up, s_up, R, split=U, x2=lo, scale2=s_lo)
        v_append(x, spec, 0, x.shape[1])
    else:
        raise StarKVError("x must be a K latent [B, H, T, R] or a V latent [B, T, R]")
    return up, s_up, lo, s_lo, R - U


def unpack_uint8_to_int4_signed(q: torch.Tensor, r: int) -> torch.Tensor:
    """[..., ceil(r/2)] uint8 nibbles -> [..., r] int8 values nibble - 8."""
    q = q.to(torch.int16)
    lo = (q & 0xF) - 8
    hi = ((q >> 4) & 0xF) - 8
    return torch.stack([lo, hi], dim=-1).flatten(-2)[..., :int(r)].to(torch.int8)
