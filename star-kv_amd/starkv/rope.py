"""RoPE configuration and device rotation tables.

Inverse frequencies follow HF ``LlamaRotaryEmbedding``: the default rule
(HF:models/llama/modeling_llama.py:103-109) and the llama3 wavelength-banded
rescale (HF:modeling_rope_utils.py:640-662).  The reference's Triton kernel
hard-codes theta=10000 without scaling (abx_rope_batched.py:184); here theta,
llama3 scaling and the attention scaling are configuration.
"""
from __future__ import annotations

import ctypes
import math
import threading
from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class RopeConfig:
    theta: float = 10000.0
    rope_type: str = "default"
    factor: float = 8.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_max_position_embeddings: int = 8192
    attention_scaling: float = 1.0
    head_dim: int = 128

    @classmethod
    def from_hf_config(cls, config) -> "RopeConfig":
        """Read theta / rope type from a transformers LlamaConfig (4.x or 5.x)."""
        params = getattr(config, "rope_parameters", None) or {}
        if not params:
            scaling = getattr(config, "rope_scaling", None) or {}
            params = dict(scaling)
            params.setdefault("rope_theta", getattr(config, "rope_theta", 10000.0))
        rtype = params.get("rope_type", params.get("type", "default")) or "default"
        kw = dict(theta=float(params.get("rope_theta", getattr(config, "rope_theta", 10000.0))),
                  rope_type=rtype)
        if rtype == "llama3":
            kw.update(factor=float(params["factor"]), low_freq_factor=float(params["low_freq_factor"]),
                      high_freq_factor=float(params["high_freq_factor"]),
                      original_max_position_embeddings=int(params["original_max_position_embeddings"]))
        elif rtype != "default":
            raise ValueError(f"rope_type {rtype!r} is not supported")
        return cls(**kw)

    def inv_freq(self) -> torch.Tensor:
        dim = self.head_dim
        inv = 1.0 / (self.theta ** (torch.arange(0, dim, 2, dtype=torch.int64).to(torch.float32) / dim))
        if self.rope_type == "default":
            return inv
        low_wl = self.original_max_position_embeddings / self.low_freq_factor
        high_wl = self.original_max_position_embeddings / self.high_freq_factor
        wavelen = 2 * math.pi / inv
        inv_l = torch.where(wavelen > low_wl, inv / self.factor, inv)
        smooth = (self.original_max_position_embeddings / wavelen - self.low_freq_factor) / (
            self.high_freq_factor - self.low_freq_factor)
        smoothed = (1 - smooth) * inv_l / self.factor + smooth * inv_l
        is_medium = ~(wavelen < high_wl) * ~(wavelen > low_wl)
        return torch.where(is_medium, smoothed, inv_l)

    def cos_sin(self, positions: torch.Tensor):
        """fp32 cos/sin [P, 128] at the given positions (HF formula)."""
        inv = self.inv_freq().to(positions.device)
        freqs = (inv[:, None] @ positions[None, :].to(torch.float32)).transpose(0, 1)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos() * self.attention_scaling, emb.sin() * self.attention_scaling


_TABLES: dict = {}
_RETIRED: list = []
_LOCK = threading.Lock()


def rope_table(cfg: RopeConfig, positions: int, device: torch.device):
    """Device rotation table covering at least `positions` positions, built
    once per (config, device) by starkv_rope_build and grown by doubling.  An
    outgrown table is retired, not freed: a captured graph keeps its address."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())    # one table per physical device
    key = (cfg, device)
    with _LOCK:
        ent = _TABLES.get(key)
        if ent is not None and ent[1] >= positions:
            return ent
        if ent is not None:
            _RETIRED.append(ent)
        cap = max(4096, 1 << max(0, (positions - 1)).bit_length())
        L = _lib.lib()
        nbytes = L.starkv_rope_table_bytes(cap)
        table = torch.empty(nbytes // 4, dtype=torch.float32, device=device)
        inv = cfg.inv_freq().contiguous()
        inv_arr = (ctypes.c_float * 64)(*inv.tolist())
        stream = torch.cuda.current_stream(device).cuda_stream
        _lib.check(L.starkv_rope_build(inv_arr, ctypes.c_float(cfg.attention_scaling), cap,
                                       ctypes.c_void_p(table.data_ptr()), nbytes, ctypes.c_void_p(stream)),
                   "starkv_rope_build")
        ent = (table, cap)
        _TABLES[key] = ent
        return ent
