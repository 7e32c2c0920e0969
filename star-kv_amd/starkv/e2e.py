"""End-to-end decode over STAR-KV latent caches (the counterpart of the
reference's ``latency.py --mode e2e``, latency.py:69-154).

A Llama-shaped ``LlamaForCausalLM`` (transformers) whose every attention is
``LatentAttention``: latent K and V projections (ragged K ranks per KV head,
one V latent per layer), a static ``LatentCache`` written in place by the HIP
cache writer (quantised on the fly), decode on ``starkv_decode_attention`` and
prefill on ``starkv_prefill_attention`` (K and V reconstructed from the cache's
latents by MFMA, then causal flash attention -- the reference materialises K
and V from the latents and calls SDPA, model.py:429-449).

The reference's e2e path replaces the attentions of a trained, exported model
(model.py:547-585) and grows its caches with ``torch.cat``
(HF:cache_utils.py:144-145); weights here are random (no checkpoints), and
HF's own cache is unused (``use_cache=False``): each layer owns its latent
cache and takes positions from it.
"""
from __future__ import annotations

import math
from typing import Callable, List, Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._lib import StarKVError
from .cache import LatentCache
from .ops import GEMM_ADD, GEMM_SILU_MUL, SKINNY_MAX_ROWS, decode_attention, prefill_attention, skinny_linear
from .rope import RopeConfig

__all__ = ["LatentAttention", "DecodeGraphState", "build_model", "fuse_layers_", "generate", "generate_graphed",
           "decode_graphed"]

HEAD_DIM = 128


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class DecodeGraphState:
    """Device-side decode position shared by every layer of a decode step
    captured once in a CUDA/HIP graph.  Each replay writes the new latents at
    ``pos`` and attends over the whole cache capacity; the decode kernels read
    ``pos`` and give the positions after it (not yet written) the logit
    -1e30.  ``advance`` runs inside the graph."""

    def __init__(self, batch: int, capacity: int, length: int, device):
        self.capacity = int(capacity)
        self.pos = torch.tensor([length], dtype=torch.int32, device=device)
        # set by the RoPE and cache-writer kernels when a replay's position
        # falls outside the capacity (they skip those rows)
        self.error = torch.zeros(1, dtype=torch.int32, device=device)

    def check(self):
        """Raise if any replay ran past the capacity (synchronises)."""
        if int(self.error.item()) != 0:
            from ._lib import StarKVError
            raise StarKVError("a graph-replayed decode step ran past the latent cache's capacity")

    def advance(self):
        self.pos.add_(1)


class LatentAttention(nn.Module):
    """One attention layer over a static latent cache.

    Weights: ``q_proj``/``o_proj`` as HF; ``k_vs`` [sum(r), hidden] (the latent K
    projection, heads back to back), ``bk`` [Hkv, r_max, 128] (B_k = k_u^T, rows
    past r_h unused), ``v_vs`` [Rv, hidden], ``v_u`` [Hkv*128, Rv] (U_v).

    ``reference = True`` runs every forward through the torch path (dequantised
    cache, K / V materialised in the act dtype as the reference does, then SDPA
    in fp32) -- the whole-model consistency reference of the kernel path."""

    def __init__(self, config, layer_idx: int, ranks: Sequence[int], v_rank: int, batch: int, capacity: int,
                 fmt: str = "int8_g64", device="cuda", dtype=torch.float16):
        super().__init__()
        self.layer_idx = layer_idx
        self.n_heads = config.num_attention_heads
        self.n_kv = config.num_key_value_heads
        if config.hidden_size // self.n_heads != HEAD_DIM or len(ranks) != self.n_kv:
            raise ValueError("LatentAttention needs head_dim 128 and one rank per KV head")
        self.ranks = [int(r) for r in ranks]
        self.rmax = max(self.ranks)
        hs = config.hidden_size
        kw = dict(device=device, dtype=dtype)
        self.q_proj = nn.Linear(hs, self.n_heads * HEAD_DIM, bias=False, **kw)
        self.o_proj = nn.Linear(self.n_heads * HEAD_DIM, hs, bias=False, **kw)
        self.k_vs = nn.Linear(hs, sum(self.ranks), bias=False, **kw)
        self.v_vs = nn.Linear(hs, v_rank, bias=False, **kw)
        self.v_u = nn.Linear(v_rank, self.n_kv * HEAD_DIM, bias=False, **kw)
        self.register_buffer("bk", torch.zeros(self.n_kv, self.rmax, HEAD_DIM, **kw))
        self.cache = LatentCache(batch, self.ranks, v_rank, capacity, dtype, device, fmt=fmt)
        self.rope = RopeConfig.from_hf_config(config)
        self.scaling = HEAD_DIM ** -0.5
        self.reference = False
        self.events: Optional[list] = None     # (start, end) CUDA events of the decode kernels, when set
        self.graph: Optional[DecodeGraphState] = None   # set: single-token forwards in graph-replay form

    def reset_parameters_(self, gen: Optional[torch.Generator] = None, std: float = 0.02):
        """Random weights of the scales a trained STAR-KV layer has: N(0, std)
        projections, B_k rows N(0, 1/r_h), U_v N(0, 1/Rv)."""
        for lin in (self.q_proj, self.o_proj, self.k_vs, self.v_vs):
            lin.weight.data.normal_(0.0, std, generator=gen)
        self.v_u.weight.data.normal_(0.0, 1.0 / math.sqrt(self.v_u.weight.shape[1]), generator=gen)
        self.bk.zero_()
        for h, r in enumerate(self.ranks):
            self.bk[h, :r].normal_(0.0, 1.0 / math.sqrt(r), generator=gen)

    @torch.no_grad()
    def load_projections(self, p) -> None:
        """Take the latent K / V projections of an exported layer
        (`starkv.export.LatentProjections`); the module must have been built
        with the same ranks and V rank."""
        if list(p.ranks) != self.ranks or p.v_vs.shape[0] != self.v_vs.weight.shape[0]:
            raise ValueError("load_projections: ranks differ from the module's")
        self.k_vs.weight.copy_(p.k_vs)
        self.bk.zero_()
        self.bk[:, :p.bk.shape[1]].copy_(p.bk)
        self.v_vs.weight.copy_(p.v_vs)
        self.v_u.weight.copy_(p.v_u)

    def _attend_torch(self, q: torch.Tensor, S: int, T: int) -> torch.Tensor:
        """q [B, Hq, T, 128] (rotated) against positions [0, S) of the cache."""
        B = q.shape[0]
        gs = self.n_heads // self.n_kv
        xk = self.cache.dequant_k(S)
        cos, sin = self.rope.cos_sin(torch.arange(S, device=q.device))
        ks = []
        for h in range(self.n_kv):
            kh = torch.matmul(xk[h], self.bk[h, :self.ranks[h]].contiguous())      # [B, S, 128]
            ks.append(kh * cos.to(kh.dtype) + _rotate_half(kh) * sin.to(kh.dtype))
        K = torch.stack(ks, 1)                                                      # [B, Hkv, S, 128]
        V = F.linear(self.cache.dequant_v(S), self.v_u.weight).view(B, S, self.n_kv, HEAD_DIM).transpose(1, 2)
        K = K.repeat_interleave(gs, 1)
        V = V.repeat_interleave(gs, 1)
        if self.reference:
            qf, Kf, Vf = q.float(), K.float().contiguous(), V.float().contiguous()
        else:
            qf, Kf, Vf = q, K.contiguous(), V.contiguous()
        if T == 1:
            o = F.scaled_dot_product_attention(qf, Kf, Vf, scale=self.scaling)
        elif T == S:
            o = F.scaled_dot_product_attention(qf, Kf, Vf, is_causal=True, scale=self.scaling)
        else:
            m = torch.ones(T, S, dtype=torch.bool, device=q.device).tril(S - T)
            o = F.scaled_dot_product_attention(qf, Kf, Vf, attn_mask=m, scale=self.scaling)
        return o.to(q.dtype)

    def merge_projections_(self) -> None:
        """Hold q_proj, k_vs and v_vs as row blocks of one weight ``qkv_weight``
        (the three Linear weights become views of it), so the projections of
        the layer input run as one GEMM; the Linear modules keep working."""
        with torch.no_grad():
            w = torch.cat([self.q_proj.weight, self.k_vs.weight, self.v_vs.weight], 0).contiguous()
        self.register_buffer("qkv_weight", w, persistent=False)
        rows = [self.q_proj.weight.shape[0], self.k_vs.weight.shape[0], self.v_vs.weight.shape[0]]
        off = 0
        for lin, n in zip((self.q_proj, self.k_vs, self.v_vs), rows):
            lin.weight = nn.Parameter(w[off:off + n], requires_grad=False)
            off += n

    def _project(self, hidden_states: torch.Tensor, rms_eps: Optional[float] = None):
        """(q [B, Hq, T, 128], new K latent rows [B, T, sum(r)], new V latent rows [B, T, Rv]).
        ``rms_eps``: hidden_states is the raw layer input and the input RMSNorm
        is folded into the packed projection (``qkv_packed``)."""
        B, T, _ = hidden_states.shape
        if rms_eps is not None:
            nq, nk = self.n_heads * HEAD_DIM, sum(self.ranks)
            qkv = skinny_linear(hidden_states, self.qkv_packed, rms_eps=rms_eps)
            return (qkv[..., :nq].view(B, T, self.n_heads, HEAD_DIM).transpose(1, 2), qkv[..., nq:nq + nk],
                    qkv[..., nq + nk:])
        w = getattr(self, "qkv_weight", None)
        if w is None or self.reference:
            q = self.q_proj(hidden_states)
            return (q.view(B, T, self.n_heads, HEAD_DIM).transpose(1, 2), self.k_vs(hidden_states),
                    self.v_vs(hidden_states))
        nq, nk = self.n_heads * HEAD_DIM, sum(self.ranks)
        if B * T <= SKINNY_MAX_ROWS and hidden_states.shape[-1] % 64 == 0 and w.shape[0] % 16 == 0:
            qkv = skinny_linear(hidden_states, w)                 # decode: one weight stream
        else:
            qkv = F.linear(hidden_states, w)
        return (qkv[..., :nq].view(B, T, self.n_heads, HEAD_DIM).transpose(1, 2), qkv[..., nq:nq + nk],
                qkv[..., nq + nk:])

    def forward(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None, past_key_values=None,
                use_cache=False, position_embeddings=None, **kwargs):
        B, T, _ = hidden_states.shape
        o = self.core(hidden_states, position_embeddings)
        return self.o_proj(o), None

    def core(self, hidden_states: torch.Tensor, position_embeddings=None,
             rms_eps: Optional[float] = None) -> torch.Tensor:
        """The attention of the layer input without the output projection: [B, T, Hq*128]
        (``rms_eps``: as in ``_project``)."""
        B, T, _ = hidden_states.shape
        q, k_new, v_new = self._project(hidden_states, rms_eps)
        # k_new [B, T, sum(r)]: the writer takes the heads packed.  The cache
        # writes and the query rotation (positions continuing the cache) run as
        # one launch
        if self.reference:
            cos, sin = position_embeddings
            q = q * cos.unsqueeze(1) + _rotate_half(q) * sin.unsqueeze(1)
        elif self.graph is not None and T == 1:
            kspec, vspec = self.cache.append_at(k_new, v_new, self.bk, self.graph.pos, error_flag=self.graph.error,
                                                q=q, rope=self.rope)
            o = decode_attention(q[:, :, 0], kspec, vspec, self.v_u.weight, rope=self.rope,
                                 seq_len=self.graph.capacity, scale=self.scaling, last_pos=self.graph.pos)
            return o.unsqueeze(1).reshape(B, T, self.n_heads * HEAD_DIM)
        if self.reference:
            kspec, vspec, S = self.cache.append(k_new, v_new, self.bk)
        else:
            kspec, vspec, S = self.cache.append(k_new, v_new, self.bk, q=q, rope=self.rope)
        if T > 1 and not self.reference:
            o = prefill_attention(q, kspec, vspec, self.v_u.weight, rope=self.rope, pos0=S - T,
                                  scale=self.scaling).transpose(1, 2)               # [B, T, Hq, 128]
        elif T == 1 and not self.reference:
            if self.events is not None:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
            o = decode_attention(q[:, :, 0], kspec, vspec, self.v_u.weight, rope=self.rope, seq_len=S,
                                 scale=self.scaling)
            if self.events is not None:
                e1.record()
                self.events.append((e0, e1))
            o = o.unsqueeze(1)                                                      # [B, 1, Hq, 128]
        else:
            o = self._attend_torch(q, S, T).transpose(1, 2)                         # [B, T, Hq, 128]
        return o.reshape(B, T, self.n_heads * HEAD_DIM)


def _fused_decoder_forward(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None,
                           past_key_values=None, use_cache=False, position_embeddings=None, **kwargs):
    """LlamaDecoderLayer.forward (transformers models/llama/modeling_llama.py)
    with the layer's own elementwise work in single launches: RMSNorm on
    ``starkv_rms_norm``, the residual adds folded into the o_proj and down_proj
    GEMMs (one rounding instead of two), gate and up projections as one GEMM
    followed by SiLU(gate) * up.  Decode batches (at most 16 rows) run the
    projections on ``starkv_skinny_gemm`` (the residual add and the SiLU
    product in its epilogue); larger ones on torch's GEMMs (addmm) and
    ``starkv_silu_mul``.  The reference path (``self_attn.reference``) runs
    HF's own forward."""
    from .ops import rms_norm, silu_mul
    att = self.self_attn
    if att.reference:
        return type(self).forward(self, hidden_states, attention_mask=attention_mask, position_ids=position_ids,
                                  past_key_values=past_key_values, use_cache=use_cache,
                                  position_embeddings=position_embeddings, **kwargs)
    _refresh_layer_(self)
    if _recording_hidden_states():
        # HF keeps each layer's output (and the embedding) as the hidden
        # states it returns: update a copy, not the tensor it recorded
        hidden_states = hidden_states.clone()
    B, T, Hd = hidden_states.shape
    eps_in, eps_post = self.input_layernorm.variance_epsilon, self.post_attention_layernorm.variance_epsilon
    if B * T <= SKINNY_MAX_ROWS and getattr(self.mlp, "gate_up_packed", None) is not None:
        # decode: four weight streams, the norms folded into the projections
        # that follow them, the residual adds and SiLU(gate) * up in epilogues
        if not hidden_states.is_contiguous():
            hidden_states = hidden_states.contiguous()
        o = att.core(hidden_states, position_embeddings, rms_eps=eps_in)
        h = hidden_states.view(-1, Hd)
        skinny_linear(o.reshape(B * T, -1), att.o_packed, out=h, epilogue=GEMM_ADD)
        m = skinny_linear(h, self.mlp.gate_up_packed, epilogue=GEMM_SILU_MUL, rms_eps=eps_post)
        skinny_linear(m, self.mlp.down_packed, out=h, epilogue=GEMM_ADD)
        return h.view(B, T, Hd)
    x = rms_norm(hidden_states, self.input_layernorm.weight, eps_in)
    o = att.core(x, position_embeddings)
    # the residual stream is updated in place (an out-of-place addmm first
    # copies its input): the layer input is the previous layer's output or
    # the embedding lookup, which nothing reads after this layer
    h = hidden_states.reshape(-1, Hd)
    if h.data_ptr() != hidden_states.data_ptr() or not h.is_contiguous():
        h = h.clone()
    o = o.reshape(B * T, -1)
    w_o, w_gu, w_d = att.o_proj.weight, self.mlp.gate_up_weight, self.mlp.down_proj.weight
    skinny = (B * T <= SKINNY_MAX_ROWS and all(t.shape[1] % 64 == 0 and t.shape[0] % 32 == 0 and t.stride(1) == 1
                                                 for t in (w_o, w_gu, w_d)))
    if skinny:
        skinny_linear(o, w_o, out=h, epilogue=GEMM_ADD)
    else:
        h.addmm_(o, w_o.t())
    n = rms_norm(h, self.post_attention_layernorm.weight, eps_post)
    if skinny:
        skinny_linear(skinny_linear(n, w_gu, epilogue=GEMM_SILU_MUL), w_d, out=h, epilogue=GEMM_ADD)
    else:
        h.addmm_(silu_mul(F.linear(n, w_gu)), w_d.t())
    return h.view(B, T, Hd)


def _fused_norm_forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
    """LlamaRMSNorm.forward in one launch (``starkv_rms_norm``); HF's own
    forward while ``starkv_reference`` is set (``generate(reference=True)``)."""
    from .ops import rms_norm
    if getattr(self, "starkv_reference", False):
        return type(self).forward(self, hidden_states)
    return rms_norm(hidden_states, self.weight, self.variance_epsilon)


def _fused_lm_head_forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
    """nn.Linear forward of the output projection on ``starkv_skinny_gemm``
    (packed weight) for decode batches, torch's GEMM otherwise."""
    if _signature((self.weight,)) != getattr(self, "_starkv_sig", None):
        _no_capture("the output projection's weight")
        self.packed = _pack_head(self)
        self._starkv_sig = _signature((self.weight,))
    rows = hidden_states.numel() // hidden_states.shape[-1]
    if rows <= SKINNY_MAX_ROWS and getattr(self, "packed", None) is not None:
        return skinny_linear(hidden_states.contiguous(), self.packed)
    return F.linear(hidden_states, self.weight, self.bias)


def _packable(w: torch.Tensor) -> bool:
    return w.dim() == 2 and w.shape[0] % 32 == 0 and w.shape[1] % 64 == 0


def _recording_hidden_states() -> bool:
    """True while HF collects every decoder layer's output
    (``output_hidden_states=True``: transformers' output-capturing hooks,
    active through a context variable); True as well when that mechanism is
    not found (another transformers version), so no recorded tensor is ever
    updated in place."""
    try:
        from transformers.utils.output_capturing import _active_collector
    except ImportError:
        return True
    col = _active_collector.get()
    return col is not None and "hidden_states" in col


def _signature(ts) -> tuple:
    """Identity and in-place version of each tensor: it changes when a weight
    is replaced or written (``load_state_dict``, ``load_projections``)."""
    return tuple((t.data_ptr(), t._version) for t in ts)


def _layer_sources(layer) -> tuple:
    att, mlp = layer.self_attn, layer.mlp
    return (att.q_proj.weight, att.k_vs.weight, att.v_vs.weight, layer.input_layernorm.weight, att.o_proj.weight,
            mlp.gate_proj.weight, mlp.up_proj.weight, layer.post_attention_layernorm.weight, mlp.down_proj.weight)


def _no_capture(what: str) -> None:
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise StarKVError(f"{what} changed since its packed copy was made: run one step eagerly (which repacks) "
                          "before capturing a graph")


def _fuse_layer_(layer) -> None:
    """Merge and pack one decoder layer's weights (see ``fuse_layers_``) and
    record the signature of the weights they were made from."""
    from .ops import pack_weight
    att = layer.self_attn
    att.merge_projections_()
    mlp = layer.mlp
    with torch.no_grad():
        w = torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight], 0).contiguous()
    mlp.register_buffer("gate_up_weight", w, persistent=False)
    n = mlp.gate_proj.weight.shape[0]
    mlp.gate_proj.weight = nn.Parameter(w[:n], requires_grad=False)
    mlp.up_proj.weight = nn.Parameter(w[n:], requires_grad=False)
    mlp.gate_up_packed = None
    # qkv rows need 16 (tiles), the others 32 (gate/up halves), k 64
    if (att.qkv_weight.shape[0] % 16 == 0 and att.qkv_weight.shape[1] % 64 == 0
            and all(_packable(t) for t in (att.o_proj.weight, w, mlp.down_proj.weight))):
        with torch.no_grad():
            att.qkv_packed = pack_weight(att.qkv_weight, layer.input_layernorm.weight)
            att.o_packed = pack_weight(att.o_proj.weight)
            mlp.gate_up_packed = pack_weight(w, layer.post_attention_layernorm.weight)
            mlp.down_packed = pack_weight(mlp.down_proj.weight)
    layer._starkv_sig = _signature(_layer_sources(layer))


def _refresh_layer_(layer) -> None:
    """Re-merge and repack a layer whose weights changed after
    ``fuse_layers_`` (the merged and packed copies would otherwise keep the
    old values); refused inside a graph capture."""
    if _signature(_layer_sources(layer)) != getattr(layer, "_starkv_sig", None):
        _no_capture("a decoder layer's weight")
        _fuse_layer_(layer)


def _pack_head(head):
    from .ops import pack_weight
    with torch.no_grad():
        return pack_weight(head.weight)


def fuse_layers_(model) -> None:
    """Run every decoder layer of ``model`` (and the final norm) through
    ``_fused_decoder_forward``: q / k / v latent projections and the MLP's
    gate / up projections merged into one weight each (the HF Linear weights
    become views of them, so HF's forward still works), the norms and
    activation on the library's kernels.  For decode batches each layer's
    four projections also get a packed copy for ``starkv_skinny_gemm``
    (``pack_weight``), the input and post-attention RMSNorm weights folded
    into the q/k/v and gate/up copies.  Each layer (and the output
    projection) records the version of the weights its copies come from and
    rebuilds them when a weight has been replaced or written since
    (``load_state_dict``, ``load_projections``)."""
    import types
    for layer in model.model.layers:
        _fuse_layer_(layer)
        layer.forward = types.MethodType(_fused_decoder_forward, layer)
    model.model.norm.forward = types.MethodType(_fused_norm_forward, model.model.norm)
    head = model.lm_head
    head.packed = None
    if _packable(head.weight) and head.bias is None:
        head.packed = _pack_head(head)
        head._starkv_sig = _signature((head.weight,))
        head.forward = types.MethodType(_fused_lm_head_forward, head)


def build_model(n_layers: int, hidden: int, heads: int, kv_heads: int, intermediate: int, vocab: int,
                ranks: Sequence[int], v_rank: int, batch: int, capacity: int, fmt: str = "int8_g64",
                seed: int = 0, device="cuda", dtype=torch.float16, projections: Optional[Sequence] = None,
                fused: bool = True):
    """Random-init LlamaForCausalLM with every attention replaced by LatentAttention.

    `projections`: per layer, an exported `LatentProjections` whose ranks and
    weights replace `ranks`, `v_rank` and the random latent projections.
    `fused`: run the decoder layers through ``fuse_layers_`` (HF's own layer
    forward otherwise; the reference path always uses HF's)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=intermediate,
                      num_hidden_layers=n_layers, num_attention_heads=heads, num_key_value_heads=kv_heads,
                      max_position_embeddings=max(4096, capacity), tie_word_embeddings=False)
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device(device):
            model = LlamaForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    model.eval()
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    for i, layer in enumerate(model.model.layers):
        p = projections[i] if projections is not None else None
        r, rv = (p.ranks, p.v_vs.shape[0]) if p is not None else (ranks, v_rank)
        att = LatentAttention(cfg, i, r, rv, batch, capacity, fmt=fmt, device=device, dtype=dtype)
        att.reset_parameters_(gen)
        if p is not None:
            att.load_projections(p)
        layer.self_attn = att
    if fused:
        fuse_layers_(model)
    return model


def attention_layers(model) -> List[LatentAttention]:
    return [layer.self_attn for layer in model.model.layers]


@torch.no_grad()
def generate(model, prompt: torch.Tensor, steps: int, reference: bool = False,
             forced: Optional[torch.Tensor] = None):
    """Greedy decoding: prefill ``prompt`` [B, P] (one forward), then ``steps``
    single-token decode forwards.  ``forced`` [B, steps] feeds given tokens
    instead of the argmax (teacher forcing, for comparing two runs).
    Returns (tokens [B, steps + 1], logits of the last position per forward)."""
    for att in attention_layers(model):
        att.reference = reference
    model.model.norm.starkv_reference = reference
    B, P = prompt.shape
    dev = prompt.device
    out = model(input_ids=prompt, position_ids=torch.arange(P, device=dev)[None].expand(B, P),
                use_cache=False, logits_to_keep=1)
    logits = [out.logits[:, -1].float()]
    tok = logits[-1].argmax(-1, keepdim=True)
    toks = [tok]
    for t in range(steps):
        inp = forced[:, t:t + 1] if forced is not None else tok
        pos = torch.full((B, 1), P + t, device=dev, dtype=torch.long)
        out = model(input_ids=inp, position_ids=pos, use_cache=False, logits_to_keep=1)
        logits.append(out.logits[:, -1].float())
        tok = logits[-1].argmax(-1, keepdim=True)
        toks.append(tok)
    return torch.cat(toks, 1), logits


@torch.no_grad()
def generate_graphed(model, prompt: torch.Tensor, steps: int, keep_logits: bool = True):
    """``generate`` with the decode steps replayed from one captured graph
    (``decode_graphed``).  Returns (tokens [B, steps + 1], logits of the last
    position per forward, or [] when ``keep_logits`` is False)."""
    for att in attention_layers(model):
        att.reference = False
    model.model.norm.starkv_reference = False
    B, P = prompt.shape
    dev = prompt.device
    out = model(input_ids=prompt, position_ids=torch.arange(P, device=dev)[None].expand(B, P),
                use_cache=False, logits_to_keep=1)
    logits = [out.logits[:, -1].float()] if keep_logits else []
    tok = out.logits[:, -1].argmax(-1, keepdim=True)
    if steps == 0:
        return tok, logits
    toks, more = decode_graphed(model, tok, steps, keep_logits)
    return torch.cat([tok, toks], 1), logits + more


@torch.no_grad()
def decode_graphed(model, tok: torch.Tensor, steps: int, keep_logits: bool = True,
                   on_step: Optional[Callable[[int], None]] = None):
    """``steps`` greedy decode steps from token ``tok`` [B, 1] at the caches'
    current length: the first step runs eagerly in graph form (which also
    warms up every table and workspace), one step is captured, and the rest
    replay it, each step's argmax feeding the next inside the graph.
    ``on_step(i)`` (optional) runs on the host after step i (0: the eager
    one) has been enqueued, e.g. to read what the step wrote.  Returns
    (tokens [B, steps], logits per step or [])."""
    atts = attention_layers(model)
    B = tok.shape[0]
    dev = tok.device
    P = atts[0].cache.length
    cap = atts[0].cache.cap
    if any(a.cache.cap != cap or a.cache.length != P for a in atts) or P + steps > cap:
        raise ValueError("decode_graphed: every layer's cache must hold the decode steps")
    state = DecodeGraphState(B, cap, P, dev)
    for att in atts:
        att.reference = False
        att.graph = state
    tok_buf = tok.clone()
    pos_buf = torch.full((B, 1), P, device=dev, dtype=torch.long)
    logit_buf = None
    toks, logits = [], []

    def step():
        # the decode forward of LlamaForCausalLM (embedding, decoder layers,
        # final norm, output projection of the last position) without HF's
        # per-forward position, mask and rotary bookkeeping: the latent
        # attentions take their positions from the graph state
        nonlocal logit_buf
        h = model.model.embed_tokens(tok_buf)
        for layer in model.model.layers:
            h = layer(h, attention_mask=None, position_ids=pos_buf, position_embeddings=None)
        last = model.lm_head(model.model.norm(h)[:, -1])
        if keep_logits:
            if logit_buf is None:
                logit_buf = torch.empty(B, last.shape[-1], device=dev, dtype=torch.float32)
            logit_buf.copy_(last)
        tok_buf.copy_(last.argmax(-1, keepdim=True))   # fp16 -> fp32 is exact: the same argmax
        state.advance()
        pos_buf.add_(1)

    try:
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            step()                                    # first decode step, eager, graph form
        torch.cuda.current_stream(dev).wait_stream(side)
        if keep_logits:
            logits.append(logit_buf.clone())
        toks.append(tok_buf.clone())
        if on_step is not None:
            on_step(0)
        if steps > 1:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            for i in range(1, steps):
                graph.replay()
                if keep_logits:
                    logits.append(logit_buf.clone())
                toks.append(tok_buf.clone())
                if on_step is not None:
                    on_step(i)
    finally:
        for att in atts:
            att.graph = None
            att.cache.length = P + steps
    state.check()
    return torch.cat(toks, 1), logits
