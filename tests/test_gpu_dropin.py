"""GPU tests of the reference-interface drop-ins (abx, LlamaCustomAttention).

Compared with the fp64 oracle (tests/_util.py, oracle/) or with an fp64
re-computation of the whole module on the CPU, on seeded inputs.
"""
import math
import sys

import pytest
import torch

from _util import check_logits, check_output, errors

HEAD = 128


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------- abx

@pytest.mark.gpu
@pytest.mark.parametrize("dtype,Hq,Hkv,S,r,theta", [
    (torch.float16, 32, 32, 300, 64, 10000.0),
    (torch.bfloat16, 8, 2, 1000, 40, 10000.0),
    (torch.float16, 4, 1, 77, 128, 500000.0),
])
def test_abx_matches_oracle(dtype, Hq, Hkv, S, r, theta):
    from oracle import starkv_oracle as o
    from starkv import RopeConfig
    from starkv.abx_rope_batched import abx
    _flush(f"[abx] {dtype} Hq={Hq} Hkv={Hkv} S={S} r={r} theta={theta}")
    g = torch.Generator(device="cuda").manual_seed(11)
    B = 3
    a = torch.randn(B, Hq, 1, HEAD, generator=g, device="cuda").to(dtype)
    b = (torch.randn(Hkv, r, HEAD, generator=g, device="cuda") / math.sqrt(r)).to(dtype)
    x = torch.randn(B, Hkv, S, r, generator=g, device="cuda").to(dtype)
    rope = RopeConfig(theta=theta) if theta == 10000.0 else RopeConfig(
        theta=theta, rope_type="llama3", factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
        original_max_position_embeddings=8192)
    out = abx(a, b, x, dtype=dtype, rope=rope)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, 1, S) and out.dtype == dtype
    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)
    ref = o.k_logits(a[:, :, 0].cpu(), [b[h].cpu() for h in range(Hkv)], [x[:, h].cpu() for h in range(Hkv)],
                     cos, sin, scale=1.0)
    _flush(f"   ref_rms={ref.pow(2).mean().sqrt().item():.3f}")
    # abx returns unscaled logits in the act dtype (abx_rope_batched.py:157): gated
    # at the softmax input's scale (bf16 against the bf16-rounded oracle) ...
    check_logits(out[:, :, 0], ref, 1.0, "act-dtype out: ")
    # ... and the same kernel's fp32 logits, which bf16 storage would otherwise mask
    from starkv import KLatentSpec, k_logits
    out32 = k_logits(a, KLatentSpec.from_reference(x, b), S, rope=rope, scale=1.0, out_dtype=torch.float32)
    check_logits(out32, ref, 1.0, "fp32 out: ")


# ---------------------------------------------------------------- attention module

class _KProj(torch.nn.Module):
    def __init__(self, vs, u):
        super().__init__()
        self.VS = vs
        self.register_buffer("U", u)


class _VProj(torch.nn.Module):
    def __init__(self, vs, u):
        super().__init__()
        self.VS = vs
        self.U = u


def _module(Hq, Hkv, r, Rv, dtype, seed=0):
    from transformers import LlamaConfig
    from starkv.LlamaLoRaAttention_headwise import LlamaCustomAttention
    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=Hq * HEAD, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      intermediate_size=256, num_hidden_layers=1, max_position_embeddings=4096)
    m = LlamaCustomAttention(cfg, layer_idx=0, decomp_goup_num=Hq)
    hid = cfg.hidden_size
    k_vs = torch.nn.Linear(hid, Hkv * r, bias=False)
    k_u = torch.randn(Hkv, HEAD, r) / math.sqrt(r)
    v_vs = torch.nn.Linear(hid, Rv, bias=False)
    v_u = torch.nn.Linear(Rv, Hkv * HEAD, bias=False)
    m.k_proj = _KProj(k_vs, k_u)
    m.v_proj = _VProj(v_vs, v_u)
    return cfg, m.to(device="cuda", dtype=dtype).eval()


def _module_reference(m, cfg, hidden_all, n_prefill):
    """fp64 CPU re-computation of every output row of the module for the
    token stream `hidden_all` [B, T, hid]: causal attention over per-position
    RoPE keys K = RoPE(X_k U_k^T) and values V = X_v U_v^T (GQA by q // gs)."""
    from oracle import starkv_oracle as o
    d = torch.float64
    h = hidden_all.cpu().to(d)
    W = lambda lin: lin.weight.detach().cpu().to(d)
    B, T, _ = h.shape
    Hq, Hkv = m.num_heads, m.num_key_value_heads
    gs = Hq // Hkv
    q = (h @ W(m.q_proj).T).view(B, T, Hq, HEAD).transpose(1, 2)
    xk = (h @ W(m.k_proj.VS).T).view(B, T, Hkv, -1).transpose(1, 2)           # [B, Hkv, T, r]
    xv = h @ W(m.v_proj.VS).T                                                 # [B, T, Rv]
    ku = m.k_proj.U.detach().cpu().to(d)                                      # [Hkv, 128, r]
    uv = W(m.v_proj.U).view(Hkv, HEAD, -1)                                    # [Hkv, 128, Rv]
    cos, sin = [t.to(d) for t in o.rope_cos_sin(m.rope.inv_freq(), torch.arange(T))]
    q = o.apply_rope(q, cos, sin)
    K = o.apply_rope(xk @ ku.transpose(-1, -2), cos, sin).repeat_interleave(gs, 1)
    V = (xv[:, None] @ uv.transpose(-1, -2)).repeat_interleave(gs, 1)         # [B, Hq, T, 128]
    att = (q @ K.transpose(-1, -2)) / math.sqrt(HEAD)
    att = att.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf")).softmax(-1)
    out = (att @ V).transpose(1, 2).reshape(B, T, -1)
    return out @ W(m.o_proj).T


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,r,Rv,dtype", [(4, 4, 48, 200, torch.float16), (8, 2, 64, 256, torch.bfloat16)])
def test_attention_module_prefill_then_decode(Hq, Hkv, r, Rv, dtype):
    """The module's attention cores (its HIP prefill and decode calls) against
    the fp64 oracle on the same inputs -- the rotated queries and the caches
    as the module stored them -- at max-abs 2e-2 / mean-rel 1e-3 (bf16 against
    the bf16-rounded oracle).  For fp16 the module output (after o_proj) is
    also held to the same gates against an fp64 re-computation of the whole
    module from its weights (the fp16 projections round at 2^-11, well inside
    them); in bf16 the projections' own rounding (2^-9) sets that error, so
    only the attention cores are gated."""
    import starkv.LlamaLoRaAttention_headwise as mod
    from transformers.cache_utils import DynamicCache
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    from _util import KernelRecorder
    _flush(f"[module] Hq={Hq} Hkv={Hkv} r={r} Rv={Rv} {dtype}")
    cfg, m = _module(Hq, Hkv, r, Rv, dtype)
    rot = LlamaRotaryEmbedding(config=cfg).to("cuda")
    B, P, n_dec = 2, 45, 3
    g = torch.Generator(device="cuda").manual_seed(5)
    hidden_all = (torch.randn(B, P + n_dec, cfg.hidden_size, generator=g, device="cuda") * 0.5).to(dtype)
    ref = _module_reference(m, cfg, hidden_all, P)
    cache = DynamicCache()
    outs = []
    with torch.no_grad(), KernelRecorder(mod) as rec:
        pos = torch.arange(P, device="cuda")[None].expand(B, P)
        pe = rot(hidden_all[:, :P], pos)
        outs.append(m(hidden_all[:, :P], pe, None, pos, past_key_values=cache)[0])
        for t in range(P, P + n_dec):
            pos = torch.full((B, 1), t, device="cuda")
            pe = rot(hidden_all[:, t:t + 1], pos)
            outs.append(m(hidden_all[:, t:t + 1], pe, None, pos, past_key_values=cache)[0])
    assert [c["kind"] for c in rec.calls] == ["prefill"] + ["decode"] * n_dec
    assert rec.check() == 1 + n_dec
    if dtype == torch.float16:
        check_output(outs[0], ref[:, :P], "module prefill output: ")
        for i, t in enumerate(range(P, P + n_dec)):
            check_output(outs[1 + i], ref[:, t:t + 1], f"module decode t={t} output: ")


@pytest.mark.gpu
@pytest.mark.parametrize("B,S", [(4, 1024), (1, 262144)])
def test_abx_reference_check_and_bench_shape(B, S):
    """The reference's own abx shapes (abx_rope_batched.py:254-280): total
    rank int(0.2 * 4096) = 819 over 32 query heads in KV groups of 4, i.e.
    8 KV heads of rank 819 // 8 = 102 (not a multiple of 8), fp16; b passed
    with one row per query head as the check does ([32, 102, 128], rows
    q // 4 read).  B4 S1024 is the check (run_test, 254-270); B1 S262144 the
    longest benchmark context (target_seq_lens, 280), checked on 2048 sampled
    positions (each logit depends on its own position only)."""
    from oracle import starkv_oracle as o
    from starkv import RopeConfig
    from starkv.abx_rope_batched import abx
    Hq, gs = 32, 4
    Hkv, r = Hq // gs, int(4096 * 0.2) // (Hq // gs)
    assert r == 102
    _flush(f"[abx reference shape] B={B} S={S} Hq={Hq} Hkv={Hkv} r={r} fp16")
    g = torch.Generator(device="cuda").manual_seed(13)
    a = torch.randn(B, Hq, 1, HEAD, generator=g, device="cuda").half()
    b = (torch.randn(Hq, r, HEAD, generator=g, device="cuda") / math.sqrt(r)).half()
    x = torch.randn(B, Hkv, S, r, generator=g, device="cuda").half()
    out = abx(a, b, x, dtype=torch.float16)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, 1, S) and out.dtype == torch.float16
    rope = RopeConfig()
    if S <= 4096:
        pos = torch.arange(S)
    else:
        pos = torch.cat([torch.arange(32), torch.randperm(S - 64, generator=torch.Generator().manual_seed(1))[:1984] + 32,
                         torch.arange(S - 32, S)]).sort().values
    cos, sin = o.rope_cos_sin(rope.inv_freq(), pos, rope.attention_scaling)
    ref = o.k_logits(a[:, :, 0].cpu(), [b[h].cpu() for h in range(Hkv)],
                     [x[:, h, pos.cuda()].cpu() for h in range(Hkv)], cos, sin, scale=1.0)
    check_logits(out[:, :, 0, pos.cuda()], ref, 1.0, "fp16 out: ")
