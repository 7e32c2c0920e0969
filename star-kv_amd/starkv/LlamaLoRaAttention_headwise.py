"""Drop-in for ``LlamaLoRaAttention_headwise.LlamaCustomAttention`` on libstarkv.

Same constructor, weights and forward signature as the reference module
(LlamaLoRaAttention_headwise.py:32-148) and the unified prefill/decode forward
the reference installs on it (model.py:387-491):

* ``q_proj`` / ``o_proj``: ``nn.Linear``;
* ``k_proj`` with ``.VS`` (``nn.Linear`` [Hkv*r, hidden]) and ``.U`` (buffer
  [Hkv, 128, r]); ``v_proj`` with ``.VS`` (``nn.Linear`` [Rv, hidden]) and
  ``.U`` (``nn.Linear``, weight [Hkv*128, Rv]) -- the inference wrappers of
  model.py:365-380, installed after construction exactly as there;
* ``forward(hidden_states, position_embeddings, attention_mask, position_ids,
  past_key_values=None, cache_position=None, **kwargs) -> (out, None)``.

Decode (one query position) runs the fused kernel chain of
``starkv_decode_attention`` (K logits with per-position RoPE, softmax, P.Xv,
per-KV-head up-projection) on the latent caches as ``past_key_values.update``
returns them: keys [B, Hkv, S, r], values [B, S, Rv].  Prefill without a mask
(HF passes none when there is no padding) runs causally on
``starkv_prefill_attention`` (K and V reconstructed from the latent caches by
MFMA, flash attention) when the caches meet its layout (ranks and strides
multiples of 8); with a mask, or another layout, it materialises K and V and
runs torch SDPA, as the reference does (model.py:429-449), causally when no
mask is given (the reference omits ``is_causal``).

Differences kept on purpose: keys are rotated by their own positions (the
reference's torch branch uses the last position for all keys,
LlamaLoRaAttention_headwise.py:22-29), and GQA is handled in decode and
prefill (the reference module's up-projection is MHA-only, 126-133).
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._lib import StarKVError
from .ops import KLatentSpec, decode_attention, prefill_attention
from .rope import RopeConfig

# the reference module's switches (LlamaLoRaAttention_headwise.py:16-19);
# decode here always takes the fused low-rank path
reorder = True
triton_kernel = True


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _prefill_layout_ok(k: torch.Tensor, v: torch.Tensor, uv: torch.Tensor) -> bool:
    """Whether starkv_prefill_attention takes the caches (dense fp16 / bf16
    latents with contiguous last dims; any rank, stride or alignment -- the
    library repacks what its kernels cannot read in place).  Other caches keep
    the reference's torch route."""
    return (k.dim() == 4 and v.dim() == 3 and k.dtype == v.dtype == uv.dtype and k.dtype in (torch.float16, torch.bfloat16)
            and k.stride(3) == 1 and v.stride(2) == 1 and uv.stride(1) == 1)


def _additive(mask: Optional[torch.Tensor], dtype: torch.dtype) -> Optional[torch.Tensor]:
    """HF hands boolean (keep = True) or additive float masks; the kernels take additive ones."""
    if mask is None or mask.dtype != torch.bool:
        return mask
    return torch.zeros(mask.shape, dtype=dtype, device=mask.device).masked_fill_(~mask, float("-inf"))


class LlamaCustomAttention(nn.Module):
    """Llama attention over a low-rank latent KV cache (decode on MI355X HIP kernels)."""

    def __init__(self, config, layer_idx: Optional[int] = None, decomp_goup_num: Optional[int] = 1):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.attention_dropout = config.attention_dropout
        self.hidden_size = config.hidden_size
        self.num_heads = config.num_attention_heads
        self.head_dim = self.hidden_size // self.num_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_key_value_groups = self.num_heads // self.num_key_value_heads
        self.max_position_embeddings = config.max_position_embeddings
        self.rope_theta = getattr(config, "rope_theta", 10000.0)
        self.is_causal = True
        self.scaling = self.head_dim ** -0.5
        self.q_proj = nn.Linear(self.hidden_size, self.num_heads * self.head_dim, bias=config.attention_bias)
        self.k_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=config.attention_bias)
        self.v_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=config.attention_bias)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, self.hidden_size, bias=config.attention_bias)
        self.decomp_goup_num = decomp_goup_num
        self.decomp_goup_num_kv = decomp_goup_num // self.num_key_value_groups
        self.rope = RopeConfig.from_hf_config(config)
        self._bk = None          # (k_u data_ptr, version, contiguous k_u^T)

    def _k_basis(self, k_u: torch.Tensor) -> torch.Tensor:
        """k_u^T [Hkv, r, 128] made contiguous once per weight version."""
        key = (k_u.data_ptr(), k_u._version, k_u.dtype)
        if self._bk is None or self._bk[0] != key:
            self._bk = (key, k_u.transpose(-2, -1).contiguous())
        return self._bk[1]

    def forward(self, hidden_states: torch.Tensor, position_embeddings, attention_mask: Optional[torch.Tensor],
                position_ids: Optional[torch.LongTensor] = None, past_key_values=None,
                cache_position: Optional[torch.LongTensor] = None, **kwargs):
        if self.head_dim != 128:
            raise StarKVError("the decode kernels are built for head_dim 128")
        input_shape = hidden_states.shape[:-1]
        query_len = input_shape[-1]
        q = self.q_proj(hidden_states).view(*input_shape, -1, self.head_dim).transpose(1, 2)
        k_u, k_vs = self.k_proj.U, self.k_proj.VS
        v_u, v_vs = self.v_proj.U, self.v_proj.VS
        k_inter = (torch.matmul(hidden_states, k_vs.weight.T)
                   .view(*input_shape, self.decomp_goup_num_kv, -1).transpose(1, 2))
        v_inter = torch.matmul(hidden_states, v_vs.weight.T)
        if past_key_values is not None:
            key_states, value_states = past_key_values.update(k_inter, v_inter, self.layer_idx)
        else:
            key_states, value_states = k_inter, v_inter

        cos, sin = position_embeddings
        c, s = cos.unsqueeze(1), sin.unsqueeze(1)
        q = q * c + _rotate_half(q) * s
        S = key_states.shape[-2]
        mask = _additive(attention_mask, q.dtype)

        if query_len > 1 and mask is None and _prefill_layout_ok(key_states, value_states, v_u.weight):
            # causal prefill on the HIP kernels: K / V reconstructed from the
            # latent caches by MFMA, then flash attention
            spec = KLatentSpec.from_reference(key_states, self._k_basis(k_u))
            out = prefill_attention(q, spec, value_states, v_u.weight, rope=self.rope, pos0=S - query_len,
                                    scale=self.scaling)
        elif query_len > 1:
            pos = torch.arange(S, device=q.device)
            kc, ks = self.rope.cos_sin(pos)
            K = torch.matmul(key_states, k_u.transpose(-2, -1).to(key_states.dtype))
            K = (K * kc.to(K.dtype) + _rotate_half(K) * ks.to(K.dtype)).repeat_interleave(self.num_key_value_groups, 1)
            V = (torch.matmul(value_states, v_u.weight.T).view(*value_states.shape[:-1], self.num_key_value_heads,
                                                                self.head_dim).transpose(-3, -2))
            V = V.repeat_interleave(self.num_key_value_groups, 1)
            if mask is not None:
                out = F.scaled_dot_product_attention(q, K, V, attn_mask=mask[:, :, :, :S], scale=self.scaling)
            else:
                causal = torch.ones(query_len, S, dtype=torch.bool, device=q.device).tril(S - query_len)
                out = F.scaled_dot_product_attention(q, K, V, attn_mask=causal, scale=self.scaling)
        else:
            spec = KLatentSpec.from_reference(key_states, self._k_basis(k_u))
            m = mask[:, :, :, :S] if mask is not None else None
            out = decode_attention(q, spec, value_states, v_u.weight, rope=self.rope, seq_len=S, mask=m,
                                   scale=self.scaling).unsqueeze(2)
        out = out.transpose(1, 2).reshape(*input_shape, -1).contiguous()
        return self.o_proj(out), None
