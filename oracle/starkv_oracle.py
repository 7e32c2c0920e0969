"""CPU oracle for the STAR-KV fused low-rank decode-attention path.

TEST INFRASTRUCTURE ONLY.  This module is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path (``star-kv_amd/``) never calls
into it and raises when its HIP library is missing.

It restates, op for op and in float64/float32 on the CPU, the eager PyTorch
decode path of the reference:

* key reconstruction + per-position RoPE + q.K^T:
  ``torch_abx`` (abx_rope_batched.py:189-202) with ``b`` indexed per *KV* head
  as the Triton kernel does (abx_rope_batched.py:81, 89) and as the model passes
  it (model.py:455);
* RoPE tables: HF ``LlamaRotaryEmbedding`` (HF:models/llama/modeling_llama.py:
  103-127), llama3 inverse-frequency scaling (HF:modeling_rope_utils.py:
  640-662), ``rotate_half`` (HF:models/llama/modeling_llama.py:130-134);
* the softmax join: ``/sqrt(D)``, ``+mask``, ``softmax(dtype=fp32)``
  (model.py:458-470);
* the "reorder" value path: ``P @ Xv`` then the per-KV-head up-projection
  (model.py:482-487);
* the prefill branch: K / V materialised from the latents, GQA repeat and
  SDPA (model.py:429-449), under the causal mask HF passes it;
* the quantised-cache formats (numpy, integer exact): the reference's int4
  nibble convention (bx_quant.py:75-86) and the build's own int8 / int4-g64
  formats (the reference's ``quant_utils`` is absent, bx_quant.py:18).

How each function is pinned (tests/test_oracle.py):

* ``rope_inv_freq`` / ``rope_cos_sin``: committed fixtures written by
  tests/golden/make_rope_fixtures.py with the installed transformers 5.15.0
  (default theta=1e4 and llama3 theta=5e5); plus closed forms (inv_freq[0]=1,
  cos^2+sin^2=1).
* ``k_logits``: (a) r=128, B_k=I reduces to textbook RoPE attention logits,
  checked against a complex-exponential formulation written independently;
  (b) ragged ranks equal zero-padded dense ranks exactly; (c) GQA head
  mapping q -> q // gs; (d) brute force in pure-Python loops on tiny S, r.
* ``decode_attention``: torch ``scaled_dot_product_attention`` on fully
  materialised K and V (the reorder identity (P Xv) Uv^T == P (Xv Uv^T),
  LlamaLoRaAttention_headwise.py:16, 126-142).
* ``reconstruct_kv`` / ``prefill_attention``: torch SDPA with
  ``is_causal=True`` on K / V materialised per query head (pos0 = 0);
  chunked prefill (pos0 > 0) equals the matching rows of the full prefill;
  the last query's row equals ``decode_attention``; planted off-by-one mask
  and transposed V head layout are caught.
* int4 unpack (reference convention): hand-computed known answers for chosen
  bytes (nibble order, bias 8) and the exhaustive 256-byte table against an
  arithmetic (divmod) decomposition; dequant rounding against torch's own
  fp16 multiply (the reference's ``torch_bx`` expression, bx_quant.py:171-172).
* build-defined quantisers (int8 symmetric, int4 asymmetric group-64):
  parity unpinned (the reference's quantiser is missing); pinned only by
  invariants: |x - deq(q(x))| <= s/2 (+ fp16 rounding), range, idempotence.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence

import numpy as np
import torch

HEAD_DIM = 128


# --------------------------------------------------------------------------
# RoPE
# --------------------------------------------------------------------------

def rope_inv_freq(theta: float = 10000.0, dim: int = HEAD_DIM, rope_type: str = "default",
                  factor: float = 8.0, low_freq_factor: float = 1.0, high_freq_factor: float = 4.0,
                  original_max_position_embeddings: int = 8192) -> torch.Tensor:
    """Inverse frequencies, fp32 [dim/2].

    default: HF:models/llama/modeling_llama.py:103-109 ->
      1 / theta ** (arange(0, dim, 2).float() / dim)
    llama3:  HF:modeling_rope_utils.py:640-662 (wavelength-banded rescale).
    """
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.int64).to(torch.float32) / dim))
    if rope_type == "default":
        return inv
    if rope_type != "llama3":
        raise ValueError(f"unsupported rope_type {rope_type!r}")
    low_wl = original_max_position_embeddings / low_freq_factor
    high_wl = original_max_position_embeddings / high_freq_factor
    wavelen = 2 * math.pi / inv
    inv_l = torch.where(wavelen > low_wl, inv / factor, inv)
    smooth = (original_max_position_embeddings / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    smoothed = (1 - smooth) * inv_l / factor + smooth * inv_l
    is_medium = ~(wavelen < high_wl) * ~(wavelen > low_wl)
    return torch.where(is_medium, smoothed, inv_l)


def rope_cos_sin(inv_freq: torch.Tensor, positions: torch.Tensor, attention_scaling: float = 1.0):
    """fp32 cos/sin [S, dim] exactly as HF computes them before the dtype cast
    (HF:models/llama/modeling_llama.py:113-127): freqs = inv_freq (x) pos in
    fp32, emb = cat(freqs, freqs), cos = emb.cos() * scaling."""
    freqs = (inv_freq[:, None].to(torch.float32) @ positions[None, :].to(torch.float32)).transpose(0, 1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos() * attention_scaling, emb.sin() * attention_scaling


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """HF:models/llama/modeling_llama.py:130-134."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x*cos + rotate_half(x)*sin with one angle per row (per position).

    This is abx_rope_batched.py:22-29 without its last-position shortcut
    (lines 25-27), i.e. the semantics of torch_abx (198-200) and _abx_fwd
    (117-125): key s is rotated by the angle of position s."""
    return x * cos + rotate_half(x) * sin


# --------------------------------------------------------------------------
# Decode path
# --------------------------------------------------------------------------

def k_logits(q: torch.Tensor, bk: Sequence[torch.Tensor], xk: Sequence[torch.Tensor],
             cos: torch.Tensor, sin: torch.Tensor, scale: float = 1.0,
             dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """Logits [B, Hq, S] = scale * q_rot . RoPE_s(Xk[s] @ Bk).

    q:  [B, Hq, D] rotated query (the ``a`` argument of abx, abx_rope_batched.py:135)
    bk: per KV head [r_h, D]  (``b`` = k_u^T, model.py:455)
    xk: per KV head [B, S, r_h] (the K latent cache, one tensor per head so
        head-wise ranks may differ)
    Query head ``qh`` reads KV head ``qh // gs`` (abx_rope_batched.py:81).
    """
    B, Hq, D = q.shape
    Hkv = len(bk)
    gs = Hq // Hkv
    S = xk[0].shape[1]
    out = torch.empty(B, Hq, S, dtype=dtype)
    c = cos[:S].to(dtype)
    s = sin[:S].to(dtype)
    qd = q.to(dtype)
    for h in range(Hkv):
        K = xk[h].to(dtype) @ bk[h].to(dtype)           # [B, S, D]   abx_rope_batched.py:191-194
        K = apply_rope(K, c, s)                         # per position   (198-200)
        for g in range(gs):
            qh = h * gs + g
            out[:, qh, :] = (K @ qd[:, qh, :, None])[..., 0] * scale   # a @ xb^T (201)
    return out


def softmax_join(logits: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """model.py:467-470: logits (already / sqrt(D)) + mask, softmax over S."""
    if mask is not None:
        logits = logits + mask.to(logits.dtype)
    return torch.softmax(logits, dim=-1)


def pv_latent(p: torch.Tensor, xv: torch.Tensor) -> torch.Tensor:
    """model.py:484: prob_v = P @ Xv -> [B, Hq, Rv]."""
    return p @ xv.to(p.dtype)


def up_proj(o_lat: torch.Tensor, uv_weight: torch.Tensor, n_kv: int) -> torch.Tensor:
    """model.py:485-487: v_u.weight [Hkv*D, Rv] viewed [Hkv, D, Rv], repeated
    per query-head group; out[b, q] = Uv[q // gs] @ o_lat[b, q] -> [B, Hq, D]."""
    B, Hq, Rv = o_lat.shape
    gs = Hq // n_kv
    U = uv_weight.to(o_lat.dtype).view(n_kv, HEAD_DIM, Rv).repeat_interleave(gs, dim=0)  # [Hq, D, Rv]
    return torch.einsum("bqr,qdr->bqd", o_lat, U)


def decode_attention(q, bk, xk, xv, uv_weight, cos, sin, mask=None, dtype=torch.float64):
    """Full decode step of the attention core (the scope of latency.py:262-268):
    logits -> softmax -> P.Xv -> up-projection.  Returns (out [B,Hq,D], P, o_lat)."""
    logits = k_logits(q, bk, xk, cos, sin, scale=1.0 / math.sqrt(HEAD_DIM), dtype=dtype)
    p = softmax_join(logits, mask)
    o_lat = pv_latent(p, xv)
    out = up_proj(o_lat, uv_weight, len(bk))
    return out, p, o_lat


# --------------------------------------------------------------------------
# Prefill path
# --------------------------------------------------------------------------

def reconstruct_kv(bk: Sequence[torch.Tensor], xk: Sequence[torch.Tensor], xv: torch.Tensor,
                   uv_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, dtype=torch.float64):
    """Materialised K and V of the reference's prefill (model.py:431-444):
    key_full = RoPE_s(X_k[s] @ B_k) per KV head (k_u^T, 431-432) and
    value_full = (X_v @ U_v^T) viewed [B, S, Hkv, D] -> [B, Hkv, S, D]
    (438-442).  Returns (K, V), both [B, Hkv, S, D] (before the GQA repeat)."""
    Hkv = len(bk)
    B, S, Rv = xv.shape
    c, s = cos[:S].to(dtype), sin[:S].to(dtype)
    K = torch.stack([apply_rope(xk[h].to(dtype) @ bk[h].to(dtype), c, s) for h in range(Hkv)], dim=1)
    V = (xv.to(dtype) @ uv_weight.to(dtype).t()).view(B, S, Hkv, HEAD_DIM).transpose(1, 2)
    return K, V


def prefill_attention(q: torch.Tensor, bk, xk, xv, uv_weight, cos, sin, pos0: int = 0,
                      scale: Optional[float] = None, dtype=torch.float64,
                      kv_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Causal prefill over the latent caches: queries q [B, Hq, T, D] (already
    rotated) at positions pos0 .. pos0+T-1; query t attends to keys
    s <= pos0 + t of the first pos0 + T cached positions.  This is the
    reference's prefill (model.py:429-449: materialise, repeat_interleave over
    the GQA group, SDPA with scale) under HF's causal attention mask.
    ``kv_dtype``: round the materialised K (after RoPE) and V once to this
    dtype before the attention, as the reference materialises key_full and
    value_full in the activation dtype (model.py:431-442).
    Returns [B, Hq, T, D]."""
    B, Hq, T, D = q.shape
    S = pos0 + T
    K, V = reconstruct_kv(bk, [x[:, :S] for x in xk], xv[:, :S], uv_weight, cos, sin, dtype)
    if kv_dtype is not None:
        K, V = K.to(kv_dtype).to(dtype), V.to(kv_dtype).to(dtype)
    gs = Hq // len(bk)
    K = K.repeat_interleave(gs, dim=1)
    V = V.repeat_interleave(gs, dim=1)
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    logits = (q.to(dtype) @ K.transpose(-1, -2)) * sc                     # [B, Hq, T, S]
    logits = logits.masked_fill(~causal_visible(T, S, pos0), float("-inf"))
    return torch.softmax(logits, dim=-1) @ V


def causal_visible(T: int, S: int, pos0: int) -> torch.Tensor:
    """[T, S] bool: query t (position pos0 + t) sees key s iff s <= pos0 + t
    (HF's causal mask, the mask the reference's SDPA call expects from its
    caller, model.py:445-449)."""
    return torch.arange(S)[None, :] <= (pos0 + torch.arange(T))[:, None]


def uniform_heads(x: torch.Tensor) -> List[torch.Tensor]:
    """Split the reference cache layout [B, Hkv, S, r] into per-head [B, S, r]."""
    return [x[:, h] for h in range(x.shape[1])]


# --------------------------------------------------------------------------
# Quantised-cache formats (numpy, integer exact)
# --------------------------------------------------------------------------

def _f16_round(x64: np.ndarray) -> np.ndarray:
    """Round float64 values (exact here) to fp16 once, round-to-nearest-even."""
    return x64.astype(np.float16)


def unpack_int4_ref(packed: np.ndarray, r: int) -> np.ndarray:
    """Reference int4 nibble convention (bx_quant.py:75-86): rank j lives in
    byte j >> 1, the low nibble for even j and the high nibble for odd j;
    value = nibble - 8.  Returns int8 [..., r]."""
    p = packed.astype(np.int16)
    lo = (p & 0x0F) - 8
    hi = ((p >> 4) & 0x0F) - 8
    out = np.stack([lo, hi], axis=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
    return out[..., :r].astype(np.int8)


def pack_int4_ref(vals: np.ndarray) -> np.ndarray:
    """Inverse of unpack_int4_ref for vals in [-8, 7]; odd r padded with 0 (-> nibble 8)."""
    v = vals.astype(np.int16) + 8
    if v.shape[-1] % 2:
        v = np.concatenate([v, np.full(v.shape[:-1] + (1,), 8, np.int16)], axis=-1)
    return (v[..., 0::2] | (v[..., 1::2] << 4)).astype(np.uint8)


def dequant_int4_ref(packed: np.ndarray, scale: np.ndarray, r: int) -> np.ndarray:
    """(nibble-8) * s rounded once to fp16 (bx_quant.py:86; torch_bx 171-172).
    scale: fp16 broadcastable to [..., r] (per token: [..., 1])."""
    n = unpack_int4_ref(packed, r).astype(np.float64)
    return _f16_round(n * scale.astype(np.float64))


def quant_int4_ref(x: np.ndarray):
    """Build's quantiser for the reference int4 format (parity unpinned: the
    reference's quantize_r_split_int8_int4_packed is missing).  Per-token
    symmetric: s = fp16(amax / 7); n = clip(rint(x / s), -8, 7)."""
    x32 = x.astype(np.float32)
    amax = np.abs(x32).max(axis=-1, keepdims=True)
    s = (amax / 7.0).astype(np.float16)
    s = np.where(s == 0, np.float16(1.0), s)
    n = np.clip(np.rint(x32 / s.astype(np.float32)), -8, 7).astype(np.int8)
    return pack_int4_ref(n), s


def quant_int8_sym(x: np.ndarray):
    """int8 symmetric with one fp16 scale per row (last axis reduced):
    s = fp16(amax / 127), q = clip(rint(x / s), -127, 127).  Build-defined
    (config 3 K latent; the reference's int8 quantiser is missing)."""
    x32 = x.astype(np.float32)
    amax = np.abs(x32).max(axis=-1, keepdims=True)
    s = (amax / 127.0).astype(np.float16)
    s = np.where(s == 0, np.float16(1.0), s)
    q = np.clip(np.rint(x32 / s.astype(np.float32)), -127, 127).astype(np.int8)
    return q, s


def dequant_int8_sym(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """fp16(q * s): exact product rounded once (…_quant.py:138 semantics)."""
    return _f16_round(q.astype(np.float64) * s.astype(np.float64))


def quant_int4_asym(x: np.ndarray, group: int = 64):
    """int4 asymmetric, groups of ``group`` along the last axis (the last group
    may be shorter): zero = fp16(min), scale = fp16((max - min) / 15),
    n = clip(rint((x - zero) / scale), 0, 15).  Build-defined (config 3 V)."""
    x32 = x.astype(np.float32)
    R = x32.shape[-1]
    G = (R + group - 1) // group
    n = np.empty(x32.shape, np.uint8)
    sc = np.empty(x32.shape[:-1] + (G,), np.float16)
    zr = np.empty(x32.shape[:-1] + (G,), np.float16)
    for g in range(G):
        blk = x32[..., g * group:(g + 1) * group]
        lo = blk.min(axis=-1)
        hi = blk.max(axis=-1)
        z = lo.astype(np.float16)
        s = ((hi - z.astype(np.float32)) / 15.0).astype(np.float16)
        s = np.where(s == 0, np.float16(1.0), s)
        q = np.rint((blk - z.astype(np.float32)[..., None]) / s.astype(np.float32)[..., None])
        n[..., g * group:(g + 1) * group] = np.clip(q, 0, 15).astype(np.uint8)
        sc[..., g] = s
        zr[..., g] = z
    return n, sc, zr


def dequant_int4_asym(n: np.ndarray, sc: np.ndarray, zr: np.ndarray, group: int = 64) -> np.ndarray:
    """fp16(n * scale + zero) rounded once from the exact value (float64 holds
    n*s + z exactly for 4-bit n and fp16 s, z)."""
    R = n.shape[-1]
    gidx = np.arange(R) // group
    s = sc.astype(np.float64)[..., gidx]
    z = zr.astype(np.float64)[..., gidx]
    return _f16_round(n.astype(np.float64) * s + z)
