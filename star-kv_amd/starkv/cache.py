"""Static latent KV caches with in-place append.

The reference grows its latent caches by ``torch.cat`` every decode step (HF
``DynamicLayer.update``, HF:cache_utils.py:127-146, reached from
model.py:411-419), re-copying the whole cache per token.  ``LatentCache``
preallocates one layer's caches for ``capacity`` positions and writes each new
token in place with the HIP cache writer (``starkv_decode_append``: the K and
V writes, with the query rotation when asked, in one launch), quantising on
the fly when the format asks for it.

Formats (K / V):
  "dense"       act dtype / act dtype
  "int8_g64"    int8 per (b, h, s) / int4 asymmetric groups of 64 per (b, s, g)
                (the quantised workload of the benchmark configurations)
  "reference"   the reference quantised module's split caches
                (LlamaLoRaAttention_headwise_quant.py:22-25, 107-127):
                K ranks [0, 16) int8 + the rest int4, V ranks [0, 256) int8 +
                the rest int4, one fp16 scale per block and token.

K is stored head-major per batch ([S_cap, r_h] per head, back to back), so
head-wise ranks may differ and each head's 32-position tile is one contiguous
run -- the layout the K-logit kernel streams best.
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import torch

from ._lib import FMT_DENSE, FMT_INT4_REF, FMT_INT8_SYM, StarKVError
from .ops import KLatentSpec, VLatentSpec, decode_append
from .rope import RopeConfig

__all__ = ["LatentCache"]

HEAD_DIM = 128


def _round(n: int, m: int) -> int:
    return (n + m - 1) // m * m


class LatentCache:
    """One layer's latent caches: K [B, Hkv, capacity, r_h], V [B, capacity, Rv]."""

    def __init__(self, batch: int, ranks: Sequence[int], v_rank: int, capacity: int, dtype: torch.dtype,
                 device, fmt: str = "dense", k_split: int = 16, v_split: int = 256):
        self.B, self.ranks, self.Rv, self.cap = int(batch), [int(r) for r in ranks], int(v_rank), int(capacity)
        self.dtype, self.device, self.fmt = dtype, torch.device(device), fmt
        self.length = 0
        Hkv, B, C = len(self.ranks), self.B, self.cap
        dev = self.device
        self._bk = None
        if fmt == "dense":
            offs = [C * sum(self.ranks[:h]) for h in range(Hkv)]
            self.k_data = torch.zeros(B, C * sum(self.ranks), dtype=dtype, device=dev)
            self._k = dict(data=self.k_data, head_offset=offs, pos_stride=self.ranks, stride_b=self.k_data.stride(0),
                           fmt=FMT_DENSE)
            self.v_data = torch.zeros(B, C, self.Rv, dtype=dtype, device=dev)
            self.v_spec = VLatentSpec.dense(self.v_data)
            return
        # scale rows padded to 8 positions: the K-logit kernel stages them in 16-byte pieces
        self.k_scale = torch.ones(B, Hkv, _round(C, 8), dtype=torch.float16, device=dev)
        if fmt == "int8_g64":
            # rows padded to 16 bytes: the K-logit kernel streams them in 16-byte pieces
            pitch = [_round(r, 16) for r in self.ranks]
            offs = [C * sum(pitch[:h]) for h in range(Hkv)]
            self.k_data = torch.zeros(B, C * sum(pitch), dtype=torch.int8, device=dev)
            self._k = dict(data=self.k_data, head_offset=offs, pos_stride=pitch, stride_b=self.k_data.stride(0),
                           fmt=FMT_INT8_SYM, scale=self.k_scale)
            G = (self.Rv + 63) // 64
            # rows padded to 16 bytes: the P.V kernel copies them in 16-byte pieces
            nb = (self.Rv + 1) // 2
            self._v_rows = torch.zeros(B, C, _round(nb, 16), dtype=torch.uint8, device=dev)
            self.v_data = self._v_rows[..., :nb]
            self.v_scale = torch.ones(B, C, G, dtype=torch.float16, device=dev)
            self.v_zero = torch.zeros(B, C, G, dtype=torch.float16, device=dev)
            self.v_spec = VLatentSpec.int4_g64(self.v_data, self.v_scale, self.v_zero, self.Rv)
            return
        if fmt != "reference":
            raise StarKVError(f"unknown cache format {fmt!r}")
        # K: upper k_split ranks int8 (16 bytes per row), the rest int4 nibbles
        up = [min(r, k_split) for r in self.ranks]
        lo = [max(r - k_split, 0) for r in self.ranks]
        pitch1 = [_round(u, 8) for u in up]
        pitch2 = [_round((l + 1) // 2, 4) for l in lo]
        self.k_data = torch.zeros(B, C * sum(pitch1), dtype=torch.int8, device=dev)
        self.k_data2 = torch.zeros(B, max(1, C * sum(pitch2)), dtype=torch.uint8, device=dev)
        self.k_scale2 = torch.ones(B, Hkv, C, dtype=torch.float16, device=dev)
        self._k = dict(data=self.k_data, head_offset=[C * sum(pitch1[:h]) for h in range(Hkv)], pos_stride=pitch1,
                       stride_b=self.k_data.stride(0), fmt=FMT_INT4_REF, scale=self.k_scale, split=k_split,
                       split_fmt=FMT_INT8_SYM, data2=self.k_data2,
                       head_offset2=[C * sum(pitch2[:h]) for h in range(Hkv)], pos_stride2=pitch2,
                       stride2_b=self.k_data2.stride(0), scale2=self.k_scale2)
        vu = min(self.Rv, v_split)
        self.v_data = torch.zeros(B, C, vu, dtype=torch.int8, device=dev)
        self.v_scale = torch.ones(B, C, 1, dtype=torch.float16, device=dev)
        if self.Rv > vu:
            self.v_data2 = torch.zeros(B, C, (self.Rv - vu + 1) // 2, dtype=torch.uint8, device=dev)
            self.v_scale2 = torch.ones(B, C, 1, dtype=torch.float16, device=dev)
            self.v_spec = VLatentSpec.int4_ref(self.v_data, self.v_scale, self.Rv, split=vu, x2=self.v_data2,
                                               scale2=self.v_scale2)
        else:
            self.v_spec = VLatentSpec.int8(self.v_data, self.v_scale)

    def k_spec(self, bk: torch.Tensor) -> KLatentSpec:
        """The K-latent description with B_k = k_u^T [Hkv, r_max, 128] (rows of
        head h beyond r_h unused) or a list of per-head [r_h, 128] tensors in one
        buffer."""
        k = self._k
        if bk.dim() != 3 or bk.stride(2) != 1:
            raise StarKVError("bk must be [Hkv, r, 128] with a contiguous last dim")
        sc = k.get("scale")
        sc2 = k.get("scale2")
        return KLatentSpec(k["data"], self.ranks, k["head_offset"], k["pos_stride"], k["stride_b"], bk,
                           [h * bk.stride(0) for h in range(len(self.ranks))], bk.stride(1), fmt=k["fmt"],
                           scale=sc, scale_stride_b=sc.stride(0) if sc is not None else 0,
                           scale_stride_h=sc.stride(1) if sc is not None else 0,
                           split=k.get("split", 0), split_fmt=k.get("split_fmt", FMT_INT4_REF),
                           data2=k.get("data2"), head_offset2=k.get("head_offset2"), pos_stride2=k.get("pos_stride2"),
                           stride2_b=k.get("stride2_b", 0), scale2=sc2,
                           scale2_stride_b=sc2.stride(0) if sc2 is not None else 0,
                           scale2_stride_h=sc2.stride(1) if sc2 is not None else 0)

    def k_rows(self, h: int) -> torch.Tensor:
        """Stored K rows of KV head h, [B, capacity, r_h] (the first block of
        the reference format; the padding of int8 rows excluded)."""
        k, C, r = self._k, self.cap, self.ranks[h]
        o, p = k["head_offset"][h], k["pos_stride"][h]
        return self.k_data[:, o:o + C * p].view(self.B, C, p)[..., :min(r, p)]

    # ---- stored values back in the act dtype (torch; prefill and reference paths)
    def _unpack_nibbles(self, packed: torch.Tensor, r: int) -> torch.Tensor:
        p = packed.to(torch.int16)
        n = torch.stack([p & 0xF, (p >> 4) & 0xF], dim=-1).flatten(-2)[..., :r]
        return n

    def dequant_k(self, length: Optional[int] = None) -> List[torch.Tensor]:
        """Per KV head the first ``length`` positions [B, S, r_h] in the act
        dtype, rounded once from the exact products as the kernels do."""
        S = self.length if length is None else int(length)
        B, C = self.B, self.cap
        out = []
        k = self._k
        for h, r in enumerate(self.ranks):
            if self.fmt == "dense":
                o = k["head_offset"][h]
                out.append(self.k_data[:, o:o + C * r].view(B, C, r)[:, :S])
            elif self.fmt == "int8_g64":
                q = self.k_rows(h)[:, :S].double()
                out.append((q * self.k_scale[:, h, :S, None].double()).to(self.dtype))
            else:
                up = min(r, k["split"])
                o1, p1 = k["head_offset"][h], k["pos_stride"][h]
                q = self.k_data[:, o1:o1 + C * p1].view(B, C, p1)[:, :S, :up].double()
                parts = [q * self.k_scale[:, h, :S, None].double()]
                if r > up:
                    o2, p2 = k["head_offset2"][h], k["pos_stride2"][h]
                    n = self._unpack_nibbles(self.k_data2[:, o2:o2 + C * p2].view(B, C, p2)[:, :S], r - up)
                    parts.append((n.double() - 8) * self.k_scale2[:, h, :S, None].double())
                out.append(torch.cat(parts, -1).to(self.dtype))
        return out

    def dequant_v(self, length: Optional[int] = None) -> torch.Tensor:
        """The first ``length`` positions of V [B, S, Rv] in the act dtype."""
        S = self.length if length is None else int(length)
        if self.fmt == "dense":
            return self.v_data[:, :S]
        if self.fmt == "int8_g64":
            n = self._unpack_nibbles(self.v_data[:, :S], self.Rv).double()
            G = self.v_scale.shape[-1]
            s = self.v_scale[:, :S].double().repeat_interleave(64, -1)[..., :self.Rv]
            z = self.v_zero[:, :S].double().repeat_interleave(64, -1)[..., :self.Rv]
            assert G * 64 >= self.Rv
            return (n * s + z).to(self.dtype)
        up = self.v_data.shape[-1]
        parts = [self.v_data[:, :S].double() * self.v_scale[:, :S].double()]
        if self.Rv > up:
            n = self._unpack_nibbles(self.v_data2[:, :S], self.Rv - up).double()
            parts.append((n - 8) * self.v_scale2[:, :S].double())
        return torch.cat(parts, -1).to(self.dtype)

    @staticmethod
    def _k_src(k_new: torch.Tensor):
        """(source for the writer, its position count): k_new is [B, Hkv, T, r_max]
        or [B, T, sum(ranks)] with the heads back to back."""
        if k_new.dim() == 3:
            return (k_new if k_new.stride(2) == 1 else k_new.contiguous()), k_new.shape[1]
        return (k_new if k_new.stride(3) == 1 else k_new.contiguous()), k_new.shape[2]

    def append_at(self, k_new: torch.Tensor, v_new: torch.Tensor, bk: torch.Tensor, pos: torch.Tensor,
                  error_flag: Optional[torch.Tensor] = None, q: Optional[torch.Tensor] = None,
                  rope: Optional[RopeConfig] = None):
        """Write k_new / v_new at the position held by the int32 device tensor
        ``pos`` (read when the writer kernels run, so the call can be captured in
        a CUDA/HIP graph and replayed at advancing positions); the host-side
        ``length`` is left to the caller.  Rows that would land past the
        capacity are skipped and set ``error_flag`` (int32 device tensor) to 1.
        With ``q`` [B, H, T, 128], its rows are rotated in place by ``rope`` at
        the same positions, in the same launch.  Returns the (K spec, V spec)."""
        src, T = self._k_src(k_new)
        if v_new.shape[1] != T:
            raise StarKVError("k_new and v_new must hold the same number of positions")
        ks = self.k_spec(bk)
        vsrc = v_new.contiguous() if v_new.stride(2) != 1 else v_new
        decode_append(src, ks, vsrc, self.v_spec, 0, self.cap, q=q, rope=rope or RopeConfig(), pos0_device=pos,
                      error_flag=error_flag)
        return ks, self.v_spec

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, bk: torch.Tensor, q: Optional[torch.Tensor] = None,
               rope: Optional[RopeConfig] = None):
        """Write T new positions (k_new [B, Hkv, T, r_max] or [B, T, sum(ranks)],
        v_new [B, T, Rv]) in place; with ``q`` [B, H, T, 128], its rows are
        rotated in place by ``rope`` at the new positions in the same launch.
        Returns (K spec, V spec, length) for the attention kernels."""
        src, T = self._k_src(k_new)
        if v_new.shape[1] != T:
            raise StarKVError("k_new and v_new must hold the same number of positions")
        if self.length + T > self.cap:
            raise StarKVError(f"cache full: {self.length} + {T} > capacity {self.cap}")
        ks = self.k_spec(bk)
        vsrc = v_new.contiguous() if v_new.stride(2) != 1 else v_new
        decode_append(src, ks, vsrc, self.v_spec, self.length, self.cap, q=q, rope=rope or RopeConfig())
        self.length += T
        return ks, self.v_spec, self.length
