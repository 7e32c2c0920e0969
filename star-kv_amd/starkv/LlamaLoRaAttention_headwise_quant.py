"""Drop-in for ``LlamaLoRaAttention_headwise_quant.LlamaCustomAttention`` on libstarkv.

Same constructor, weights and forward signature as the reference's quantised
module (LlamaLoRaAttention_headwise_quant.py:38-202), including its four
cache arguments ``past_key_values_upper`` / ``past_key_values_lower`` /
``scales_upper`` / ``scales_lower`` and its split: the top UPPER_RANKS_K = 16
K ranks and UPPER_RANKS_V = 256 V ranks in int8, the rest in packed int4, one
fp16 scale per block and token (22-25, 107-127).

* New latents are quantised by the HIP cache writer
  (``quant_utils.quantize_r_split_int8_int4_packed``).
* Decode (one query position) runs ``starkv_decode_attention`` on the split
  caches directly: dequantisation (bit-exact fp16), K logits with per-position
  RoPE, softmax, P.V and the per-KV-head up-projection.  The caches are not
  repeated per query head (the reference repeats them, 146-147); GQA is
  handled by the kernels.
* Causal prefill (no explicit mask) runs ``starkv_prefill_attention`` on the
  same split caches: the kernels dequantise them bit-exactly while
  reconstructing K (with RoPE) and V on MFMA, then flash attention.  With an
  explicit mask, prefill dequantises the caches and runs masked SDPA.

Keys are rotated by their own positions (the reference's no-kernel branch
uses the last position for all keys, 28-35, 142).
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._lib import StarKVError
from .LlamaLoRaAttention_headwise import _additive, _rotate_half
from .ops import KLatentSpec, VLatentSpec, decode_attention, prefill_attention
from .quant_utils import quantize_r_split_int8_int4_packed, unpack_uint8_to_int4_signed
from .rope import RopeConfig

reorder = True
triton_kernel_k = True
triton_kernel_v = True

UPPER_RANKS_K = 16
UPPER_RANKS_V = 256


class LlamaCustomAttention(nn.Module):
    """Llama attention over a quantised low-rank latent KV cache (decode and causal prefill on MI355X HIP kernels)."""

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
        self._bk = None

    def _k_basis(self, k_u: torch.Tensor) -> torch.Tensor:
        key = (k_u.data_ptr(), k_u._version, k_u.dtype)
        if self._bk is None or self._bk[0] != key:
            self._bk = (key, k_u.transpose(-2, -1).contiguous())
        return self._bk[1]

    def forward(self, hidden_states: torch.Tensor, position_embeddings, attention_mask: Optional[torch.Tensor],
                position_ids: Optional[torch.LongTensor] = None, past_key_values_upper=None,
                past_key_values_lower=None, scales_upper=None, scales_lower=None,
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
        rk, rv = k_inter.shape[-1], v_inter.shape[-1]
        ku_q, sku, kl_q, skl, r4_k = quantize_r_split_int8_int4_packed(k_inter, UPPER_RANKS_K)
        vu_q, svu, vl_q, svl, r4_v = quantize_r_split_int8_int4_packed(v_inter, UPPER_RANKS_V)
        if past_key_values_upper is not None and past_key_values_lower is not None:
            ku_q, vu_q = past_key_values_upper.update(ku_q, vu_q, self.layer_idx)
            kl_q, vl_q = past_key_values_lower.update(kl_q, vl_q, self.layer_idx)
            sku, svu = scales_upper.update(sku, svu, self.layer_idx)
            skl, svl = scales_lower.update(skl, svl, self.layer_idx)

        cos, sin = position_embeddings
        q = q * cos.unsqueeze(1) + _rotate_half(q) * sin.unsqueeze(1)
        S = ku_q.shape[-2]
        mask = _additive(attention_mask, q.dtype)

        def specs():
            kspec = KLatentSpec.from_reference_quant(ku_q, sku, self._k_basis(k_u), rk, x2=kl_q, s2=skl,
                                                     split=UPPER_RANKS_K)
            return kspec, VLatentSpec.int4_ref(vu_q, svu, rv, split=UPPER_RANKS_V, x2=vl_q, scale2=svl)

        if query_len > 1 and mask is None:
            kspec, vspec = specs()
            out = prefill_attention(q, kspec, vspec, v_u.weight, rope=self.rope, pos0=S - query_len,
                                    scale=self.scaling)
        elif query_len > 1:
            dt = q.dtype
            kx = torch.cat([(ku_q.to(torch.float32) * sku.float()).to(torch.float16),
                            (unpack_uint8_to_int4_signed(kl_q, r4_k).float() * skl.float()).to(torch.float16)], -1)
            vx = torch.cat([(vu_q.to(torch.float32) * svu.float()).to(torch.float16),
                            (unpack_uint8_to_int4_signed(vl_q, r4_v).float() * svl.float()).to(torch.float16)], -1)
            kc, ks = self.rope.cos_sin(torch.arange(S, device=q.device))
            K = torch.matmul(kx.to(dt), k_u.transpose(-2, -1).to(dt))
            K = (K * kc.to(dt) + _rotate_half(K) * ks.to(dt)).repeat_interleave(self.num_key_value_groups, 1)
            V = (torch.matmul(vx.to(dt), v_u.weight.T).view(*vx.shape[:-1], self.num_key_value_heads,
                                                            self.head_dim).transpose(-3, -2))
            V = V.repeat_interleave(self.num_key_value_groups, 1)
            am = mask[:, :, :, :S] if mask is not None else \
                torch.ones(query_len, S, dtype=torch.bool, device=q.device).tril(S - query_len)
            out = F.scaled_dot_product_attention(q, K, V, attn_mask=am, scale=self.scaling)
        else:
            kspec, vspec = specs()
            m = mask[:, :, :, :S] if mask is not None else None
            out = decode_attention(q, kspec, vspec, v_u.weight, rope=self.rope, seq_len=S, mask=m,
                                   scale=self.scaling).unsqueeze(2)
        out = out.transpose(1, 2).reshape(*input_shape, -1).contiguous()
        return self.o_proj(out), None
