"""Torch-facing operators over the libstarkv C ABI.

Tensors stay where they are (borrowed device pointers, arbitrary strides with
a contiguous last dimension); outputs and workspaces are allocated through
torch's caching allocator; work is enqueued on torch's current stream.
"""
from __future__ import annotations

import ctypes
import math
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import (BF16, F16, F32, FMT_DENSE, FMT_INT4_G64, FMT_INT4_REF, FMT_INT8_SYM, DecodeDesc, KAppendDesc,
                   PrefillDesc, RmsNormDesc, RopeApplyDesc, SiluMulDesc, SkinnyGemmDesc,
                   KLatent, KLogitsDesc, PVDesc, StarKVError, VAppendDesc, VLatent, check, i64_array, int_array)
from .rope import RopeConfig, rope_table

HEAD_DIM = 128


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return F16
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float32:
        return F32
    raise StarKVError(f"unsupported dtype {t.dtype}")


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise StarKVError("libstarkv operators take device tensors (there is no CPU path)")


_WS: dict = {}
_WS_RETIRED: list = []

# Test hook: when True, every output and workspace the operators allocate is
# filled with 0xFF bytes before the call (NaN in fp16, bf16 and fp32), so an
# element a kernel fails to write reads as NaN rather than as a stale value
# left in recycled memory.  Skipped inside a graph capture.
POISON = False


def _poison(t: torch.Tensor) -> torch.Tensor:
    if POISON and t.is_cuda and not torch.cuda.is_current_stream_capturing():
        t.view(torch.uint8).fill_(0xFF)
    return t


def _out(*shape, dtype, device) -> torch.Tensor:
    return _poison(torch.empty(*shape, dtype=dtype, device=device))


def _workspace(device, nbytes: int) -> torch.Tensor:
    """Per-device scratch reused across calls (ordered on one stream).

    A captured CUDA/HIP graph keeps the address of the workspace it was
    captured with, so a buffer that is outgrown is retired, never freed: the
    replays of an earlier graph keep writing memory that nothing else owns.
    Growing during a capture is refused (run the call once eagerly first)."""
    key = torch.device(device)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if key.type == "cuda" and torch.cuda.is_current_stream_capturing():
            raise StarKVError("the libstarkv workspace would grow inside a graph capture: run the same call "
                              "once before capturing it")
        if ws is not None:
            _WS_RETIRED.append(ws)
        ws = torch.empty(max(nbytes, 2 * ws.numel() if ws is not None else 0, 1 << 20), dtype=torch.uint8,
                         device=device)
        _WS[key] = ws
    _poison(ws[:max(nbytes, 1)])
    return ws


class KLatentSpec:
    """Where the key latent of every KV head lives (see include/starkv.h,
    starkv_klatent).  Element (b, h, s, j) is at
    data[b*stride_b + head_offset[h] + s*pos_stride[h] + j]; B_k (k_u^T) row j
    of head h at bk[bk_head_offset[h] + j*bk_row_stride]."""

    def __init__(self, data: torch.Tensor, ranks: Sequence[int], head_offset: Sequence[int],
                 pos_stride: Sequence[int], stride_b: int, bk: torch.Tensor, bk_head_offset: Sequence[int],
                 bk_row_stride: int, fmt: int = FMT_DENSE, scale: Optional[torch.Tensor] = None,
                 scale_stride_b: int = 0, scale_stride_h: int = 0, split: int = 0, split_fmt: int = FMT_INT4_REF,
                 data2: Optional[torch.Tensor] = None, head_offset2: Optional[Sequence[int]] = None,
                 pos_stride2: Optional[Sequence[int]] = None, stride2_b: int = 0,
                 scale2: Optional[torch.Tensor] = None, scale2_stride_b: int = 0, scale2_stride_h: int = 0):
        self.data, self.bk, self.scale = data, bk, scale
        self.ranks = [int(r) for r in ranks]
        self.head_offset = [int(v) for v in head_offset]
        self.pos_stride = [int(v) for v in pos_stride]
        self.stride_b = int(stride_b)
        self.bk_head_offset = [int(v) for v in bk_head_offset]
        self.bk_row_stride = int(bk_row_stride)
        self.fmt = fmt
        self.scale_stride_b, self.scale_stride_h = int(scale_stride_b), int(scale_stride_h)
        self.split, self.split_fmt = int(split), split_fmt
        self.data2, self.scale2 = data2, scale2
        n = len(self.ranks)
        self.head_offset2 = [int(v) for v in (head_offset2 or [0] * n)]
        self.pos_stride2 = [int(v) for v in (pos_stride2 or [0] * n)]
        self.stride2_b = int(stride2_b)
        self.scale2_stride_b, self.scale2_stride_h = int(scale2_stride_b), int(scale2_stride_h)

    @property
    def tensors(self):
        return [t for t in (self.data, self.bk, self.scale, self.data2, self.scale2) if t is not None]

    @property
    def n_kv_heads(self) -> int:
        return len(self.ranks)

    @classmethod
    def from_reference(cls, x: torch.Tensor, b: torch.Tensor) -> "KLatentSpec":
        """The reference layouts: x = K latent cache [B, Hkv, S, r]
        (LlamaLoRaAttention_headwise.py:88-102), b = k_u^T [Hkv, r, 128]
        (model.py:455)."""
        if x.dim() != 4 or b.dim() != 3:
            raise StarKVError("expected x [B, Hkv, S, r] and b [Hkv, r, 128]")
        B, H, S, r = x.shape
        if b.shape[0] != H or b.shape[1] != r or b.shape[2] != HEAD_DIM:
            raise StarKVError(f"b shape {tuple(b.shape)} does not match x {tuple(x.shape)}")
        if x.stride(3) != 1 or b.stride(2) != 1:
            raise StarKVError("the last dimension of x and b must be contiguous")
        return cls(x, [r] * H, [h * x.stride(1) for h in range(H)], [x.stride(2)] * H, x.stride(0),
                   b, [h * b.stride(0) for h in range(H)], b.stride(1))

    @staticmethod
    def _bk_args(b: torch.Tensor, n_heads: int):
        """B_k [Hkv_b, r, 128]; with n_heads = a multiple of Hkv_b (a latent
        cache repeated per query head, LlamaLoRaAttention_headwise_quant.py:
        146-147), latent head h uses B_k of head h // (n_heads // Hkv_b)."""
        if b.dim() != 3 or b.shape[2] != HEAD_DIM or b.stride(2) != 1 or n_heads % b.shape[0]:
            raise StarKVError("b must be [Hkv, r, 128] with a contiguous last dim")
        rep = n_heads // b.shape[0]
        return [(h // rep) * b.stride(0) for h in range(n_heads)], b.stride(1)

    @classmethod
    def from_reference_quant(cls, x1: torch.Tensor, s1: torch.Tensor, b: torch.Tensor, rank: int,
                             x2: Optional[torch.Tensor] = None, s2: Optional[torch.Tensor] = None,
                             split: Optional[int] = None) -> "KLatentSpec":
        """The quantised K cache of LlamaLoRaAttention_headwise_quant.py:107-127:
        x1 [B, H, S, split] int8 (or [B, H, S, split/2] uint8 int4 nibbles),
        s1 [B, H, S, 1] fp16, x2 [B, H, S, ceil((rank - split)/2)] uint8 int4 nibbles
        (any rank; split a multiple of 16),
        s2 [B, H, S, 1] fp16; b = k_u^T [Hkv, rank, 128] with H = Hkv or a
        multiple of it.  With x2 None, x1 holds all ranks (int8: INT8_SYM,
        uint8 nibbles: INT4_REF)."""
        if x1.dim() != 4 or s1.dim() != 4 or x1.stride(3) != 1:
            raise StarKVError("x1 must be [B, H, S, bytes] and s1 [B, H, S, 1]")
        B, H, S, w1 = x1.shape
        rank = int(rank)
        bko, bkr = cls._bk_args(b, H)
        ho, ps = [h * x1.stride(1) for h in range(H)], [x1.stride(2)] * H
        if x2 is None:
            if x1.dtype == torch.int8 and w1 == rank:
                fmt = FMT_INT8_SYM
            elif w1 == (rank + 1) // 2:
                fmt = FMT_INT4_REF
            else:
                raise StarKVError(f"x1 last dim {w1} matches neither int8 nor int4 storage of rank {rank}")
            return cls(x1, [rank] * H, ho, ps, x1.stride(0), b, bko, bkr, fmt, s1, s1.stride(0), s1.stride(1))
        split = int(split if split is not None else (w1 if x1.dtype == torch.int8 else 2 * w1))
        upper = FMT_INT8_SYM if (x1.dtype == torch.int8 and w1 == split) else FMT_INT4_REF
        if upper == FMT_INT4_REF and w1 * 2 != split:
            raise StarKVError("x1 does not hold `split` ranks")
        if x2.dim() != 4 or x2.shape[3] != (rank - split + 1) // 2 or x2.stride(3) != 1:
            raise StarKVError("x2 must be [B, H, S, ceil((rank - split)/2)]")
        return cls(x1, [rank] * H, ho, ps, x1.stride(0), b, bko, bkr, FMT_INT4_REF, s1, s1.stride(0), s1.stride(1),
                   split=split, split_fmt=upper, data2=x2, head_offset2=[h * x2.stride(1) for h in range(H)],
                   pos_stride2=[x2.stride(2)] * H, stride2_b=x2.stride(0), scale2=s2,
                   scale2_stride_b=s2.stride(0), scale2_stride_h=s2.stride(1))

    def c_struct(self, keep: list) -> KLatent:
        arrs = (int_array(self.ranks), i64_array(self.head_offset), i64_array(self.pos_stride),
                i64_array(self.bk_head_offset), i64_array(self.head_offset2), i64_array(self.pos_stride2))
        keep.extend(arrs)
        k = KLatent()
        k.n_kv_heads = self.n_kv_heads
        k.rank, k.head_offset, k.pos_stride, k.bk_head_offset = arrs[:4]
        k.stride_b = self.stride_b
        k.format = self.fmt
        k.data = self.data.data_ptr()
        k.scale = self.scale.data_ptr() if self.scale is not None else None
        k.scale_stride_b, k.scale_stride_h = self.scale_stride_b, self.scale_stride_h
        k.bk = self.bk.data_ptr()
        k.bk_row_stride = self.bk_row_stride
        k.split, k.split_format = self.split, self.split_fmt
        k.head_offset2, k.pos_stride2 = arrs[4], arrs[5]
        if self.data2 is not None:
            k.data2, k.stride2_b = self.data2.data_ptr(), self.stride2_b
        if self.scale2 is not None:
            k.scale2, k.scale2_stride_b, k.scale2_stride_h = (self.scale2.data_ptr(), self.scale2_stride_b,
                                                              self.scale2_stride_h)
        return k


def _q3(q: torch.Tensor) -> torch.Tensor:
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise StarKVError("decode takes one query token per sequence")
        q = q[:, :, 0, :]
    if q.dim() != 3 or q.shape[-1] != HEAD_DIM or q.stride(-1) != 1:
        raise StarKVError("q must be [B, Hq, 128] (or [B, Hq, 1, 128]) with a contiguous last dim")
    return q


def _mask_args(mask: Optional[torch.Tensor], B: int, S: int, Hq: int):
    """Accept an additive mask broadcastable to [B, Hq, S] (HF's [B, 1, 1, S>=S] included)."""
    if mask is None:
        return None, 0, 0, 0
    m = mask
    while m.dim() > 3:
        if m.shape[-2] != 1:
            raise StarKVError("decode masks must have one query row")
        m = m.select(-2, 0)
    if m.dim() == 2:
        m = m[:, None, :]
    if m.shape[-1] < S or m.stride(-1) != 1:
        raise StarKVError("mask must cover S positions with a contiguous last dim")
    if m.shape[0] not in (1, B) or m.shape[1] not in (1, Hq):
        raise StarKVError(f"mask of shape {tuple(mask.shape)} does not broadcast to [B={B}, Hq={Hq}, S]")
    sb = m.stride(0) if m.shape[0] == B else 0
    sh = m.stride(1) if m.shape[1] != 1 else 0
    return m, _dt(m), sb, sh


def k_logits(q: torch.Tensor, k: KLatentSpec, seq_len: int, rope: RopeConfig = RopeConfig(),
             scale: float = 1.0, mask: Optional[torch.Tensor] = None,
             out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """logits[b, q, s] = scale * q_rot[b,q] . RoPE_s(X_k[b, q//gs, s] @ B_k[q//gs]) (+ mask), [B, Hq, S]."""
    q = _q3(q)
    _require_cuda(q, mask, *k.tensors)
    B, Hq, _ = q.shape
    S = int(seq_len)
    out_dtype = out_dtype or torch.float32
    out = _out(B, Hq, S, dtype=out_dtype, device=q.device)
    table, cap = rope_table(rope, S, q.device)
    m, mdt, msb, msh = _mask_args(mask, B, S, Hq)
    keep: list = []
    d = KLogitsDesc()
    d.batch, d.n_q_heads, d.head_dim, d.seq_len = B, Hq, HEAD_DIM, S
    d.dtype = _dt(q)
    d.q, d.q_stride_b, d.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    d.k = k.c_struct(keep)
    d.rope_table, d.rope_max_positions = table.data_ptr(), cap
    d.scale = float(scale)
    d.mask = m.data_ptr() if m is not None else None
    d.mask_dtype, d.mask_stride_b, d.mask_stride_h = mdt, msb, msh
    d.out, d.out_dtype, d.out_stride_b, d.out_stride_h = out.data_ptr(), _dt(out), out.stride(0), out.stride(1)
    L = _lib.lib()
    nb = L.starkv_k_logits_workspace_bytes(ctypes.byref(d))
    ws = _workspace(q.device, nb) if nb else None
    check(L.starkv_k_logits(ctypes.byref(d), ctypes.c_void_p(ws.data_ptr()) if ws is not None else None,
                            ws.numel() if ws is not None else 0, _stream(q.device)), "starkv_k_logits")
    return out


class VLatentSpec:
    """Where the value latent lives and how it is stored (include/starkv.h,
    starkv_vlatent).  Build one with ``dense``, ``int4_ref``, ``int8`` or
    ``int4_g64``; strides are in elements of the stored type (bytes for the
    packed formats, fp16 elements for scales and zero points)."""

    def __init__(self, rank: int, fmt: int, data: torch.Tensor, scale: Optional[torch.Tensor] = None,
                 split: int = 0, split_fmt: int = FMT_INT4_REF, data2: Optional[torch.Tensor] = None,
                 scale2: Optional[torch.Tensor] = None, zero: Optional[torch.Tensor] = None):
        self.rank, self.fmt, self.data, self.scale = int(rank), fmt, data, scale
        self.split, self.split_fmt, self.data2, self.scale2, self.zero = int(split), split_fmt, data2, scale2, zero

    @property
    def tensors(self):
        return [t for t in (self.data, self.scale, self.data2, self.scale2, self.zero) if t is not None]

    @classmethod
    def dense(cls, xv: torch.Tensor) -> "VLatentSpec":
        """[B, S, Rv] act dtype (the reference cache, LlamaLoRaAttention_headwise.py:96-102)."""
        if xv.dim() != 3 or xv.stride(2) != 1:
            raise StarKVError("V latent must be [B, S, Rv] with a contiguous last dim")
        return cls(xv.shape[2], FMT_DENSE, xv)

    @classmethod
    def int4_ref(cls, x1: torch.Tensor, scale1: torch.Tensor, rank: int, split: Optional[int] = None,
                 x2: Optional[torch.Tensor] = None, scale2: Optional[torch.Tensor] = None) -> "VLatentSpec":
        """The reference's quantised V cache (bx_quant.py:117-166): ranks
        [0, split) in ``x1`` with one fp16 scale per token ``scale1`` [B, S, 1],
        ranks [split, rank) in ``x2`` / ``scale2``; ``x2`` holds int4 nibbles
        [B, S, ceil((rank - split)/2)] (rank 2k in the low nibble of byte k, value
        nibble - 8).  Any rank; split a multiple of 8 (the Triton kernel needs a
        multiple of its 64-rank block, bx_quant.py:72).  ``x1`` holds int4
        nibbles [B, S, ceil(split/2)] (the Triton
        kernel's reading, bx_quant.py:75-86) or int8 values [B, S, split] (the
        reading of LlamaLoRaAttention_headwise_quant.py:138, 164); the last
        dimension tells which."""
        split = int(rank if split is None else split)
        if x1.dim() != 3 or scale1.dim() != 3 or x1.stride(2) != 1:
            raise StarKVError("x1 must be [B, S, bytes] and its scale [B, S, 1]")
        if x1.shape[2] == split and x1.dtype == torch.int8:
            upper = FMT_INT8_SYM
        elif x1.shape[2] == (split + 1) // 2:
            upper = FMT_INT4_REF
        else:
            raise StarKVError(f"x1 last dim {x1.shape[2]} matches neither int4 ({(split + 1) // 2}) nor int8 ({split}) storage")
        if split < rank:
            if x2 is None or scale2 is None or x2.shape[2] != (rank - split + 1) // 2:
                raise StarKVError("the lower block needs x2 [B, S, ceil((rank - split)/2)] and its scales")
            return cls(rank, FMT_INT4_REF, x1, scale1, split, upper, x2, scale2)
        return cls(rank, FMT_INT4_REF if upper == FMT_INT4_REF else FMT_INT8_SYM, x1, scale1)

    @classmethod
    def int8(cls, q: torch.Tensor, scale: torch.Tensor) -> "VLatentSpec":
        """int8 [B, S, Rv] with one fp16 scale per token [B, S, 1]: x = q * s."""
        return cls(q.shape[2], FMT_INT8_SYM, q, scale)

    @classmethod
    def int4_g64(cls, packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, rank: int) -> "VLatentSpec":
        """int4 asymmetric, groups of 64 ranks: packed nibbles [B, S, rank/2]
        (rank 2k low nibble of byte k), fp16 scale and zero [B, S, ceil(rank/64)]
        with one set of strides: x = n * s + z rounded once to fp16."""
        if scale.stride() != zero.stride():
            raise StarKVError("scale and zero must share strides")
        return cls(rank, FMT_INT4_G64, packed, scale, zero=zero)

    def c_struct(self) -> VLatent:
        v = VLatent()
        v.rank, v.format = self.rank, self.fmt
        d = self.data
        v.data, v.stride_b, v.stride_s = d.data_ptr(), d.stride(0), d.stride(1)
        if self.scale is not None:
            v.scale, v.scale_stride_b, v.scale_stride_s = self.scale.data_ptr(), self.scale.stride(0), self.scale.stride(1)
        if self.data2 is not None:
            v.split, v.split_format = self.split, self.split_fmt
            v.data2, v.stride2_b, v.stride2_s = self.data2.data_ptr(), self.data2.stride(0), self.data2.stride(1)
            v.scale2, v.scale2_stride_b, v.scale2_stride_s = (self.scale2.data_ptr(), self.scale2.stride(0),
                                                              self.scale2.stride(1))
        if self.zero is not None:
            v.zero = self.zero.data_ptr()
        return v


def _vspec(xv) -> VLatentSpec:
    return xv if isinstance(xv, VLatentSpec) else VLatentSpec.dense(xv)


def pv_latent(p: torch.Tensor, xv) -> torch.Tensor:
    """out[b, h, j] = sum_s p[b, h, s] * V[b, s, j]  (model.py:484; bx_quant.py:117-166),
    [B, H, Rv] in p's dtype.  ``xv``: dense [B, S, Rv] tensor or a VLatentSpec."""
    v = _vspec(xv)
    _require_cuda(p, *v.tensors)
    if p.dim() != 3 or p.stride(2) != 1:
        raise StarKVError("p must be [B, H, S] with a contiguous last dim")
    B, H, S = p.shape
    if v.data.shape[0] != B or v.data.shape[1] < S:
        raise StarKVError("the V latent must be [B, >=S, ...]")
    out = _out(B, H, v.rank, dtype=p.dtype, device=p.device)
    d = PVDesc()
    d.batch, d.n_heads, d.seq_len, d.dtype = B, H, S, _dt(p)
    d.p, d.p_stride_b, d.p_stride_h = p.data_ptr(), p.stride(0), p.stride(1)
    d.v = v.c_struct()
    d.out, d.out_stride_b, d.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    L = _lib.lib()
    nb = L.starkv_pv_latent_workspace_bytes(ctypes.byref(d))
    ws = _workspace(p.device, nb)
    check(L.starkv_pv_latent(ctypes.byref(d), ctypes.c_void_p(ws.data_ptr()), ws.numel(), _stream(p.device)),
          "starkv_pv_latent")
    return out


def decode_attention(q: torch.Tensor, k: KLatentSpec, xv: torch.Tensor, uv_weight: torch.Tensor,
                     rope: RopeConfig = RopeConfig(), seq_len: Optional[int] = None,
                     mask: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                     out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
                     events: Optional[Sequence] = None, noalloc: bool = False,
                     last_pos: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused decode attention core (model.py:450-487): [B, Hq, 128] in q's dtype
    (or float32 with out_dtype=torch.float32).  ``events``: four
    torch.cuda.Event recorded around the three kernels (timing).
    ``noalloc``: run starkv_decode_attention_noalloc, whose workspace is the
    library's own device array (no workspace allocation; with ``out`` given
    the call allocates nothing at all).
    ``last_pos``: an int32 device tensor whose first element is read by the
    kernels: positions after it take the logit -1e30, as an additive -1e30
    mask would give them (a context length kept on the device for graph
    replay; the caller keeps it alive while the call or a captured graph runs).

    q: rotated query [B, Hq, 128]; k: key-latent spec; xv: V latent [B, S, Rv]
    (dense tensor) or a VLatentSpec; uv_weight: v_proj.U.weight [Hkv*128, Rv];
    seq_len defaults to the V latent's position count."""
    q = _q3(q)
    v = _vspec(xv)
    _require_cuda(q, uv_weight, mask, last_pos, *k.tensors, *v.tensors)
    if last_pos is not None and (last_pos.dtype != torch.int32 or last_pos.numel() < 1):
        raise StarKVError("last_pos must be an int32 device tensor with at least one element")
    B, Hq, _ = q.shape
    S = int(seq_len if seq_len is not None else v.data.shape[1])
    if uv_weight.dim() != 2 or uv_weight.stride(1) != 1 or uv_weight.shape[1] != v.rank:
        raise StarKVError("uv_weight must be [Hkv*128, Rv] with a contiguous last dim")
    if uv_weight.shape[0] != k.n_kv_heads * HEAD_DIM:
        raise StarKVError("uv_weight rows must be Hkv*128")
    if out is None:
        out = _out(B, Hq, HEAD_DIM, dtype=out_dtype or q.dtype, device=q.device)
    if out.dtype not in (q.dtype, torch.float32) or out.stride(-1) != 1:
        raise StarKVError("out must be [B, Hq, 128] of q's dtype or float32")
    table, cap = rope_table(rope, S, q.device)
    m, mdt, msb, msh = _mask_args(mask, B, S, Hq)
    keep: list = []
    d = DecodeDesc()
    d.batch, d.n_q_heads, d.head_dim, d.seq_len = B, Hq, HEAD_DIM, S
    d.dtype = _dt(q)
    d.q, d.q_stride_b, d.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    d.k = k.c_struct(keep)
    d.v = v.c_struct()
    d.uv, d.uv_row_stride = uv_weight.data_ptr(), uv_weight.stride(0)
    d.rope_table, d.rope_max_positions = table.data_ptr(), cap
    d.scale = float(scale if scale is not None else 1.0 / math.sqrt(HEAD_DIM))
    d.mask = m.data_ptr() if m is not None else None
    d.mask_dtype, d.mask_stride_b, d.mask_stride_h = mdt, msb, msh
    d.out, d.out_stride_b, d.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    d.out_dtype = F32 if out.dtype == torch.float32 else 0
    d.last_pos_device = last_pos.data_ptr() if last_pos is not None else None
    L = _lib.lib()
    if noalloc:
        if events is not None:
            raise StarKVError("the allocation-free decode has no timed form")
        check(L.starkv_decode_attention_noalloc(ctypes.byref(d), _stream(q.device)), "starkv_decode_attention_noalloc")
        return out
    nb = L.starkv_decode_workspace_bytes(ctypes.byref(d))
    if nb == 0:
        # re-run validation through the call itself to surface the status code
        check(L.starkv_decode_attention(ctypes.byref(d), None, 0, _stream(q.device)), "starkv_decode_attention")
    ws = _workspace(q.device, nb)
    if events is None:
        check(L.starkv_decode_attention(ctypes.byref(d), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                        _stream(q.device)), "starkv_decode_attention")
    else:
        for e in events:
            if e.cuda_event == 0:
                e.record()   # creates the underlying hipEvent
        handles = (ctypes.c_void_p * 4)(*[e.cuda_event for e in events])
        check(L.starkv_decode_attention_timed(ctypes.byref(d), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                              _stream(q.device), handles), "starkv_decode_attention_timed")
    return out


def prefill_attention(q: torch.Tensor, k: KLatentSpec, xv, uv_weight: torch.Tensor,
                      rope: RopeConfig = RopeConfig(), pos0: int = 0, scale: Optional[float] = None,
                      out: Optional[torch.Tensor] = None, events: Optional[Sequence] = None) -> torch.Tensor:
    """Causal prefill attention over the latent caches (the reference's prefill
    branch, model.py:429-449, with the causal mask applied): [B, Hq, T, 128]
    in q's dtype.

    q: rotated queries [B, Hq, T, 128] (last dim contiguous) at positions
    pos0 .. pos0 + T - 1; k / xv: the K and V latent caches holding at least
    pos0 + T positions (K dense, int8 or the reference split format; V dense
    [B, S, Rv] or a quantised VLatentSpec: group-64 int4, int8 or the
    reference split format); uv_weight: v_proj.U.weight [Hkv*128, Rv].  ``events``:
    three torch.cuda.Event recorded before the K / V reconstruction, after it
    and after the attention kernel (timing)."""
    if q.dim() != 4 or q.shape[-1] != HEAD_DIM or q.stride(-1) != 1:
        raise StarKVError("q must be [B, Hq, T, 128] with a contiguous last dim")
    v = _vspec(xv)
    _require_cuda(q, uv_weight, *k.tensors, *v.tensors)
    B, Hq, T, _ = q.shape
    if uv_weight.dim() != 2 or uv_weight.stride(1) != 1 or uv_weight.shape != (k.n_kv_heads * HEAD_DIM, v.rank):
        raise StarKVError("uv_weight must be [Hkv*128, Rv] with a contiguous last dim")
    if out is None:
        out = _out(B, Hq, T, HEAD_DIM, dtype=q.dtype, device=q.device)
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise StarKVError("out must be [B, Hq, T, 128] of q's dtype with a contiguous last dim")
    table, cap = rope_table(rope, int(pos0) + T, q.device)
    keep: list = []
    d = PrefillDesc()
    d.batch, d.n_q_heads, d.head_dim, d.n_tokens, d.pos0 = B, Hq, HEAD_DIM, T, int(pos0)
    d.dtype = _dt(q)
    d.q, d.q_stride_b, d.q_stride_h, d.q_stride_t = q.data_ptr(), q.stride(0), q.stride(1), q.stride(2)
    d.k = k.c_struct(keep)
    d.v = v.c_struct()
    d.uv, d.uv_row_stride = uv_weight.data_ptr(), uv_weight.stride(0)
    d.rope_table, d.rope_max_positions = table.data_ptr(), cap
    d.scale = float(scale if scale is not None else 1.0 / math.sqrt(HEAD_DIM))
    d.out, d.out_stride_b, d.out_stride_h, d.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1), out.stride(2)
    L = _lib.lib()
    nb = L.starkv_prefill_workspace_bytes(ctypes.byref(d))
    if nb == 0:
        check(L.starkv_prefill_attention(ctypes.byref(d), None, 0, _stream(q.device)), "starkv_prefill_attention")
    ws = _workspace(q.device, nb)
    if events is None:
        check(L.starkv_prefill_attention(ctypes.byref(d), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                         _stream(q.device)), "starkv_prefill_attention")
    else:
        for e in events:
            if e.cuda_event == 0:
                e.record()   # creates the underlying hipEvent
        handles = (ctypes.c_void_p * 3)(*[e.cuda_event for e in events])
        check(L.starkv_prefill_attention_timed(ctypes.byref(d), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                               _stream(q.device), handles), "starkv_prefill_attention_timed")
    return out


def rope_apply(x: torch.Tensor, rope: RopeConfig = RopeConfig(), pos0: int = 0,
               pos0_device: Optional[torch.Tensor] = None, max_positions: Optional[int] = None,
               error_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotate query rows x [B, H, T, 128] (act dtype, last dim contiguous) in
    place by the RoPE of positions pos0 + t (the query half of HF's
    apply_rotary_pos_emb, model.py:423); ``pos0_device``: an int32 device
    tensor read when the kernel runs (graph capture / replay), with
    ``max_positions`` bounding the positions it may hold; a row whose run-time
    position falls outside them is left as it is and sets ``error_flag`` (an
    int32 device tensor the caller zeroes and checks) to 1.  Returns x."""
    d = _rope_apply_desc(x, rope, pos0, pos0_device, max_positions, error_flag)
    check(_lib.lib().starkv_rope_apply(ctypes.byref(d), _stream(x.device)), "starkv_rope_apply")
    return x


def _rope_apply_desc(x, rope, pos0, pos0_device, max_positions, error_flag) -> RopeApplyDesc:
    if x.dim() != 4 or x.shape[-1] != HEAD_DIM or x.stride(-1) != 1:
        raise StarKVError("x must be [B, H, T, 128] with a contiguous last dim")
    _require_cuda(x)
    B, H, T, _ = x.shape
    table, cap = rope_table(rope, max(int(pos0) + T, int(max_positions or 0)), x.device)
    d = RopeApplyDesc()
    d.batch, d.n_heads, d.n_tokens, d.dtype = B, H, T, _dt(x)
    d.x, d.stride_b, d.stride_h, d.stride_t = x.data_ptr(), x.stride(0), x.stride(1), x.stride(2)
    d.rope_table, d.rope_max_positions = table.data_ptr(), cap
    d.pos0 = int(pos0)
    d.pos0_device = _pos_ptr(pos0_device)
    d.error_flag = _flag_ptr(error_flag)
    return d


def _flag_ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if t.dtype != torch.int32 or not t.is_cuda or t.numel() < 1:
        raise StarKVError("error_flag must be an int32 device tensor")
    return t.data_ptr()


def _cache_batch(t: torch.Tensor) -> int:
    """Batch size of a cache buffer (its leading dimension)."""
    return t.shape[0]


def k_append(src: torch.Tensor, k: KLatentSpec, pos0: int, capacity: int,
             pos0_device: Optional[torch.Tensor] = None, error_flag: Optional[torch.Tensor] = None) -> None:
    """Write the new K latent rows into the cache described by ``k`` at
    positions [pos0, pos0 + T), quantising to its format (starkv_k_append).
    src: [B, Hkv, T, >= r_h], or [B, T, sum(r_h)] with the heads back to back
    (the latent projection's own output); act dtype, last dim contiguous.
    ``pos0_device``: an int32 device tensor holding the position, read when
    the kernel runs (graph capture / replay); rows it would place outside the
    capacity are skipped and set ``error_flag`` (int32 device tensor) to 1."""
    keep: list = []
    d = _k_append_desc(src, k, pos0, capacity, pos0_device, error_flag, keep)
    check(_lib.lib().starkv_k_append(ctypes.byref(d), _stream(src.device)), "starkv_k_append")


def _k_append_desc(src, k, pos0, capacity, pos0_device, error_flag, keep) -> KAppendDesc:
    packed = src.dim() == 3
    if packed:
        if src.stride(2) != 1 or src.shape[2] < sum(k.ranks):
            raise StarKVError("packed src must be [B, T, sum(ranks)] with a contiguous last dim")
        src = src.unsqueeze(1)                       # [B, 1, T, sum(r)]: head h at a column offset
    elif src.dim() != 4 or src.stride(3) != 1:
        raise StarKVError("src must be [B, Hkv, T, r] with a contiguous last dim")
    elif src.shape[1] < k.n_kv_heads or src.shape[3] < max(k.ranks):
        raise StarKVError(f"src {tuple(src.shape)} holds fewer than {k.n_kv_heads} heads or "
                          f"{max(k.ranks)} ranks")
    if src.shape[0] > _cache_batch(k.data):
        raise StarKVError(f"src batch {src.shape[0]} exceeds the cache's {_cache_batch(k.data)}")
    _require_cuda(src, *[t for t in (k.data, k.scale, k.data2, k.scale2) if t is not None])
    d = KAppendDesc()
    d.batch, d.n_tokens, d.pos0, d.capacity, d.dtype = src.shape[0], src.shape[2], int(pos0), int(capacity), _dt(src)
    d.src, d.src_stride_b, d.src_stride_h, d.src_stride_t = src.data_ptr(), src.stride(0), src.stride(1), src.stride(2)
    d.k = k.c_struct(keep)
    if packed:
        offs = i64_array([sum(k.ranks[:h]) for h in range(k.n_kv_heads)])
        keep.append(offs)
        d.src_head_offset = offs
    d.pos0_device = _pos_ptr(pos0_device)
    d.error_flag = _flag_ptr(error_flag)
    return d


def _pos_ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if t.dtype != torch.int32 or not t.is_cuda:
        raise StarKVError("pos0_device must be an int32 device tensor")
    return t.data_ptr()


def v_append(src: torch.Tensor, v: VLatentSpec, pos0: int, capacity: int,
             pos0_device: Optional[torch.Tensor] = None, error_flag: Optional[torch.Tensor] = None) -> None:
    """Write the new V latent rows src [B, T, Rv] (act dtype, last dim
    contiguous) into the cache described by ``v`` at positions
    [pos0, pos0 + T), quantising to its format (starkv_v_append);
    ``pos0_device`` / ``error_flag`` as in ``k_append``."""
    d = _v_append_desc(src, v, pos0, capacity, pos0_device, error_flag)
    check(_lib.lib().starkv_v_append(ctypes.byref(d), _stream(src.device)), "starkv_v_append")


def _v_append_desc(src, v, pos0, capacity, pos0_device, error_flag) -> VAppendDesc:
    if src.dim() != 3 or src.stride(2) != 1:
        raise StarKVError("src must be [B, T, Rv] with a contiguous last dim")
    if src.shape[2] < v.rank:
        raise StarKVError(f"src rows hold {src.shape[2]} ranks, the cache stores {v.rank}")
    if src.shape[0] > _cache_batch(v.data):
        raise StarKVError(f"src batch {src.shape[0]} exceeds the cache's {_cache_batch(v.data)}")
    _require_cuda(src, *v.tensors)
    d = VAppendDesc()
    d.batch, d.n_tokens, d.pos0, d.capacity, d.dtype = src.shape[0], src.shape[1], int(pos0), int(capacity), _dt(src)
    d.src, d.src_stride_b, d.src_stride_t = src.data_ptr(), src.stride(0), src.stride(1)
    d.v = v.c_struct()
    d.pos0_device = _pos_ptr(pos0_device)
    d.error_flag = _flag_ptr(error_flag)
    return d


def decode_append(k_src: torch.Tensor, k: KLatentSpec, v_src: torch.Tensor, v: "VLatentSpec", pos0: int,
                  capacity: int, q: Optional[torch.Tensor] = None, rope: RopeConfig = RopeConfig(),
                  pos0_device: Optional[torch.Tensor] = None, error_flag: Optional[torch.Tensor] = None) -> None:
    """``k_append``, ``v_append`` and (when ``q`` is given) ``rope_apply`` of
    the query rows q [B, H, T, 128] at the same positions, in one launch
    (starkv_decode_append)."""
    keep: list = []
    kd = _k_append_desc(k_src, k, pos0, capacity, pos0_device, error_flag, keep)
    vd = _v_append_desc(v_src, v, pos0, capacity, pos0_device, error_flag)
    qd = (_rope_apply_desc(q, rope, pos0, pos0_device, capacity if pos0_device is not None else None, error_flag)
          if q is not None else None)
    check(_lib.lib().starkv_decode_append(ctypes.byref(kd), ctypes.byref(vd),
                                          ctypes.byref(qd) if qd is not None else None, _stream(k_src.device)),
          "starkv_decode_append")


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """t viewed as [rows, width] rows with a contiguous last dim (a copy-free view or an error)."""
    if t.stride(-1) != 1:
        raise StarKVError(f"{name} must have a contiguous last dim")
    try:
        return t.view(-1, t.shape[-1])
    except RuntimeError:
        raise StarKVError(f"{name} rows must be addressable with one row stride") from None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: Optional[torch.Tensor] = None,
             out: Optional[torch.Tensor] = None, residual_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """HF LlamaRMSNorm over the last dim in one launch (starkv_rms_norm),
    optionally after the residual add that precedes it in the decoder layer:
    x' = x + residual (stored to ``residual_out`` when given), then
    weight * (x' * rsqrt(mean(x'^2) + eps)) with HF's roundings.  Returns out."""
    _require_cuda(x, weight)
    xr = _rows(x, "x")
    H = x.shape[-1]
    if weight.shape != (H,) or weight.dtype != x.dtype or not weight.is_contiguous():
        raise StarKVError("weight must be a contiguous [hidden] tensor of x's dtype")
    if out is None:
        out = torch.empty_like(x)
    d = RmsNormDesc()
    d.rows, d.hidden, d.dtype = xr.shape[0], H, _dt(x)
    d.x, d.x_stride = xr.data_ptr(), xr.stride(0)
    for name, t in (("out", out), ("residual", residual), ("residual_out", residual_out)):
        if t is not None and (t.shape != x.shape or t.dtype != x.dtype or t.device != x.device):
            raise StarKVError(f"{name} must match x's shape, dtype and device")
    if residual_out is not None and residual is None:
        raise StarKVError("residual_out needs residual")
    orr = _rows(out, "out")
    d.out, d.out_stride = orr.data_ptr(), orr.stride(0)
    if residual is not None:
        rr = _rows(residual, "residual")
        d.residual, d.residual_stride = rr.data_ptr(), rr.stride(0)
    if residual_out is not None:
        ro = _rows(residual_out, "residual_out")
        d.residual_out, d.residual_out_stride = ro.data_ptr(), ro.stride(0)
    d.weight, d.eps = weight.data_ptr(), float(eps)
    check(_lib.lib().starkv_rms_norm(ctypes.byref(d), _stream(x.device)), "starkv_rms_norm")
    return out


def silu_mul(gate: torch.Tensor, up: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """LlamaMLP's SiLU(gate) * up in one launch (starkv_silu_mul).  With
    ``up`` None, ``gate`` holds [..., 2 I] = the gate and up halves of one
    merged projection.  Returns [..., I] in gate's dtype."""
    _require_cuda(gate)
    if up is None:
        if gate.shape[-1] % 2:
            raise StarKVError("a merged gate/up tensor has an even last dim")
        W = gate.shape[-1] // 2
        g, u = gate[..., :W], gate[..., W:]
    else:
        if up.shape != gate.shape or up.dtype != gate.dtype:
            raise StarKVError("gate and up must match in shape and dtype")
        W, g, u = gate.shape[-1], gate, up
    if out is None:
        out = torch.empty(*g.shape, dtype=gate.dtype, device=gate.device)
    if out.shape != g.shape or out.dtype != gate.dtype:
        raise StarKVError("out must be [..., I] of gate's dtype")
    gr, ur, orr = _rows(g, "gate"), _rows(u, "up"), _rows(out, "out")
    d = SiluMulDesc()
    d.rows, d.width, d.dtype = gr.shape[0], W, _dt(gate)
    d.gate, d.gate_stride = gr.data_ptr(), gr.stride(0)
    d.up, d.up_stride = ur.data_ptr(), ur.stride(0)
    d.out, d.out_stride = orr.data_ptr(), orr.stride(0)
    check(_lib.lib().starkv_silu_mul(ctypes.byref(d), _stream(gate.device)), "starkv_silu_mul")
    return out


SKINNY_MAX_ROWS = 16
GEMM_STORE, GEMM_ADD, GEMM_SILU_MUL = 0, 1, 2


def skinny_linear(x: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None,
                  epilogue: int = GEMM_STORE, rms_eps: Optional[float] = None) -> torch.Tensor:
    """nn.Linear x W^T for decode batches (at most 16 rows of x over its
    leading dims) on starkv_skinny_gemm; ``weight`` [n, k] or packed by
    ``pack_weight`` (faster: streamed linearly).  ``epilogue``: GEMM_STORE (out =
    x W^T), GEMM_ADD (out += x W^T, in place: the residual add) or
    GEMM_SILU_MUL (weight = gate rows then up rows: out = SiLU(x Wg^T) *
    (x Wu^T)).  ``rms_eps``: x is the raw input of an RMSNorm whose weight
    is folded into ``weight`` (``pack_weight(w, norm_weight)``); the products
    are scaled by rsqrt(mean(x^2) + rms_eps) per row.  Returns out [..., n]
    (n/2 for GEMM_SILU_MUL)."""
    _require_cuda(x, weight)
    xr = _rows(x, "x")
    packed = weight.dim() == 4
    if packed:
        if (weight.shape[2:] != (16, 64) or not weight.is_contiguous() or weight.shape[1] * 64 != x.shape[-1]
                or weight.dtype != x.dtype):
            raise StarKVError("a packed weight must be pack_weight's contiguous [n/16, k/64, 16, 64] of x's dtype")
        n = weight.shape[0] * 16
    elif weight.dim() != 2 or weight.stride(1) != 1 or weight.shape[1] != x.shape[-1] or weight.dtype != x.dtype:
        raise StarKVError("weight must be [n, k] of x's dtype with a contiguous last dim, k = x.shape[-1]")
    else:
        n = weight.shape[0]
    n_out = n // 2 if epilogue == GEMM_SILU_MUL else n
    if out is None:
        if epilogue == GEMM_ADD:
            raise StarKVError("GEMM_ADD accumulates into a given out")
        out = torch.empty(*x.shape[:-1], n_out, dtype=x.dtype, device=x.device)
    if out.shape != (*x.shape[:-1], n_out) or out.dtype != x.dtype:
        raise StarKVError(f"out must be [..., {n_out}] of x's dtype")
    orr = _rows(out, "out")
    d = SkinnyGemmDesc()
    d.m, d.n, d.k, d.dtype, d.epilogue = xr.shape[0], n, x.shape[-1], _dt(x), int(epilogue)
    d.x, d.x_stride = xr.data_ptr(), xr.stride(0)
    d.w, d.w_stride, d.w_packed = weight.data_ptr(), (0 if packed else weight.stride(0)), int(packed)
    d.rms, d.rms_eps = int(rms_eps is not None), float(rms_eps or 0.0)
    d.out, d.out_stride = orr.data_ptr(), orr.stride(0)
    check(_lib.lib().starkv_skinny_gemm(ctypes.byref(d), _stream(x.device)), "starkv_skinny_gemm")
    return out


def pack_weight(w: torch.Tensor, norm_weight: Optional[torch.Tensor] = None) -> torch.Tensor:
    """An nn.Linear weight [n, k] (n a multiple of 16, k of 64) in the layout
    starkv_skinny_gemm streams linearly: [n/16, k/64, 16, 64], each 16-row
    tile's 64-column block contiguous (a copy).  ``norm_weight`` [k]: the
    weight of an RMSNorm applied to the input first, folded in (w * norm_weight
    per column, rounded once to w's dtype) for ``skinny_linear(...,
    rms_eps=...)``."""
    n, k = w.shape
    if n % 16 or k % 64:
        raise StarKVError("pack_weight needs n a multiple of 16 and k of 64")
    if norm_weight is not None:
        if norm_weight.shape != (k,):
            raise StarKVError("norm_weight must be [k]")
        w = (w.float() * norm_weight.float()).to(w.dtype)
    return w.reshape(n // 16, 16, k // 64, 64).permute(0, 2, 1, 3).contiguous()
