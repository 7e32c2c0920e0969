"""GPU tests of the latent-cache writers (quantise / append in place) and the quantised module.

The writer must reproduce the oracle's quantisers bit for bit (the same fp16
input values, the same rounding steps); decode over a cache it filled must
match the oracle on the oracle-quantised history.
"""
import math
import sys

import numpy as np
import pytest
import torch

from _util import cfg2_ranks, check_output, errors

HEAD = 128


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 8, 37, 128), (3, 50, 1640)])
def test_quantize_r_split_bit_exact(shape):
    from oracle import starkv_oracle as o
    from starkv.quant_utils import quantize_r_split_int8_int4_packed, unpack_uint8_to_int4_signed
    _flush(f"[quantize split] {shape}")
    U = 16 if len(shape) == 4 else 256
    g = torch.Generator(device="cuda").manual_seed(1)
    x = (torch.randn(*shape, generator=g, device="cuda") * 3).half()
    x[..., ::11] *= 20
    x[0, 0] = 0                                               # an all-zero row: scale 1
    up, s_up, lo, s_lo, r4 = quantize_r_split_int8_int4_packed(x, U)
    torch.cuda.synchronize()
    xn = x.float().cpu().numpy()
    q8, s8 = o.quant_int8_sym(xn[..., :U])
    p4, s4 = o.quant_int4_ref(xn[..., U:])
    assert r4 == shape[-1] - U
    assert np.array_equal(up.cpu().numpy(), q8)
    assert np.array_equal(s_up.cpu().numpy().view(np.uint16), s8.view(np.uint16))
    assert np.array_equal(lo.cpu().numpy(), p4)
    assert np.array_equal(s_lo.cpu().numpy().view(np.uint16), s4.view(np.uint16))
    assert np.array_equal(unpack_uint8_to_int4_signed(lo, r4).cpu().numpy(), o.unpack_int4_ref(p4, r4))


def _oracle_history(fmt, kx, vx, ranks, Rv):
    """Oracle-quantised (then dequantised) K per head [B, S, r_h] and V [B, S, Rv] from float histories."""
    from oracle import starkv_oracle as o
    if fmt == "dense":
        return [torch.from_numpy(kx[h]).double() for h in range(len(ranks))], torch.from_numpy(vx).double()
    ks = []
    for h, r in enumerate(ranks):
        x = kx[h]
        if fmt == "int8_g64":
            q, s = o.quant_int8_sym(x)
            d = o.dequant_int8_sym(q, s)
        else:
            q, s = o.quant_int8_sym(x[..., :min(r, 16)])
            parts = [o.dequant_int8_sym(q, s)]
            if r > 16:
                p, s2 = o.quant_int4_ref(x[..., 16:])
                parts.append(o.dequant_int4_ref(p, s2, r - 16))
            d = np.concatenate(parts, axis=-1)
        ks.append(torch.from_numpy(d.astype(np.float64)))
    if fmt == "int8_g64":
        n, sc, zr = o.quant_int4_asym(vx, 64)
        v = o.dequant_int4_asym(n, sc, zr, 64)
    else:
        U = min(Rv, 256)
        q, s = o.quant_int8_sym(vx[..., :U])
        parts = [o.dequant_int8_sym(q, s)]
        if Rv > U:
            p, s2 = o.quant_int4_ref(vx[..., U:])
            parts.append(o.dequant_int4_ref(p, s2, Rv - U))
        v = np.concatenate(parts, axis=-1)
    return ks, torch.from_numpy(v.astype(np.float64))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["dense", "int8_g64", "reference"])
def test_latent_cache_append_then_decode(fmt):
    from oracle import starkv_oracle as o
    from starkv import RopeConfig, decode_attention
    from starkv.cache import LatentCache
    _flush(f"[cache] {fmt}")
    B, Rv, cap = 2, 1640, 96
    ranks = cfg2_ranks()[:8]                                  # 8 heads, ragged 16..96
    Hkv, Hq = len(ranks), 16
    rmax = max(ranks)
    g = torch.Generator(device="cuda").manual_seed(3)
    cache = LatentCache(B, ranks, Rv, cap, torch.float16, "cuda", fmt=fmt)
    bk = torch.zeros(Hkv, rmax, HEAD, device="cuda")
    for h, r in enumerate(ranks):
        bk[h, :r] = torch.randn(r, HEAD, generator=g, device="cuda") / math.sqrt(r)
    bk = bk.half()
    uv = (torch.randn(Hkv * HEAD, Rv, generator=g, device="cuda") / math.sqrt(Rv)).half()
    steps = [40, 1, 1, 1]
    kh, vh = [], []
    rope = RopeConfig()
    for T in steps:
        k_new = torch.randn(B, Hkv, T, rmax, generator=g, device="cuda").half()
        for h, r in enumerate(ranks):
            k_new[:, h, :, r:] = 0
        v_new = torch.randn(B, T, Rv, generator=g, device="cuda").half()
        v_new[..., ::37] *= 10
        kspec, vspec, S = cache.append(k_new, v_new, bk)
        kh.append(k_new.float().cpu().numpy())
        vh.append(v_new.float().cpu().numpy())
        q = torch.randn(B, Hq, HEAD, generator=g, device="cuda").half()
        out = decode_attention(q, kspec, vspec, uv, rope=rope, seq_len=S, out_dtype=torch.float32)
        torch.cuda.synchronize()
        kx = np.concatenate(kh, axis=2)
        kx = [kx[:, h, :, :r] for h, r in enumerate(ranks)]
        ks, v = _oracle_history(fmt, kx, np.concatenate(vh, axis=1), ranks, Rv)
        cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)
        ref, _, _ = o.decode_attention(q.cpu(), [bk[h, :r].cpu() for h, r in enumerate(ranks)], ks, v, uv.cpu(), cos, sin)
        mx, mr = errors(out, ref)
        _flush(f"   S={S} max_abs={mx:.3e} mean_rel={mr:.3e}")
        assert mr <= 1e-3 and mx <= 2e-2
    if fmt == "int8_g64":
        # stored bytes of head 0 equal the oracle's quantisation of its rows
        q0, s0 = o.quant_int8_sym(np.concatenate(kh, axis=2)[:, 0, :, :ranks[0]])
        stored = cache.k_rows(0)[:, :S].cpu().numpy()
        assert np.array_equal(stored, q0)
        assert np.array_equal(cache.k_scale[:, 0, :S].cpu().numpy().view(np.uint16), s0[..., 0].view(np.uint16))


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


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,r,Rv", [(8, 2, 80, 512),
                                         # the reference's own odd shapes: K rank 100 (16 + 84), V rank
                                         # int(0.3 * 4096) = 1228 (256 + 972: 486-byte int4 rows)
                                         (8, 2, 100, 1228)])
def test_quant_module_prefill_and_decode_match_dequantised_history(Hq, Hkv, r, Rv):
    from oracle import starkv_oracle as o
    from transformers import LlamaConfig
    from transformers.cache_utils import DynamicCache
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    from starkv.LlamaLoRaAttention_headwise_quant import LlamaCustomAttention
    _flush(f"[quant module] Hq={Hq} Hkv={Hkv} r={r} Rv={Rv}, prefill 33 (checked) + 3 decode steps")
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=Hq * HEAD, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      intermediate_size=256, num_hidden_layers=1, max_position_embeddings=4096)
    m = LlamaCustomAttention(cfg, layer_idx=0, decomp_goup_num=Hq)
    m.k_proj = _KProj(torch.nn.Linear(cfg.hidden_size, Hkv * r, bias=False), torch.randn(Hkv, HEAD, r) / math.sqrt(r))
    m.v_proj = _VProj(torch.nn.Linear(cfg.hidden_size, Rv, bias=False), torch.nn.Linear(Rv, Hkv * HEAD, bias=False))
    m = m.to(device="cuda", dtype=torch.float16).eval()
    rot = LlamaRotaryEmbedding(config=cfg).to("cuda")
    B, P = 2, 33
    g = torch.Generator(device="cuda").manual_seed(4)
    hid = (torch.randn(B, P + 3, cfg.hidden_size, generator=g, device="cuda") * 0.5).half()
    caches = [DynamicCache() for _ in range(4)]

    def dequantised():
        """The module's own caches, dequantised: K [B, Hkv, S, r], V [B, S, Rv]."""
        ku, vu = caches[0].layers[0].keys, caches[0].layers[0].values
        kl, vl = caches[1].layers[0].keys, caches[1].layers[0].values
        sku, svu = caches[2].layers[0].keys, caches[2].layers[0].values
        skl, svl = caches[3].layers[0].keys, caches[3].layers[0].values
        kx = np.concatenate([o.dequant_int8_sym(ku.cpu().numpy(), sku.cpu().numpy()),
                             o.dequant_int4_ref(kl.cpu().numpy(), skl.cpu().numpy(), r - 16)], -1)
        vx = np.concatenate([o.dequant_int8_sym(vu.cpu().numpy(), svu.cpu().numpy()),
                             o.dequant_int4_ref(vl.cpu().numpy(), svl.cpu().numpy(), Rv - 256)], -1)
        return kx, vx

    bk = m.k_proj.U.double().cpu().transpose(-1, -2)
    with torch.no_grad():
        pos = torch.arange(P, device="cuda")[None].expand(B, P)
        pre, _ = m(hid[:, :P], rot(hid[:, :P], pos), None, pos, *caches)
        torch.cuda.synchronize()
        # causal prefill (the HIP prefill kernels): fp64 causal attention over
        # the dequantised caches, K and V rounded once to fp16 as the module
        # materialises them in its dtype
        kx, vx = dequantised()
        q = (hid[:, :P].double().cpu() @ m.q_proj.weight.double().cpu().T).view(B, P, Hq, HEAD).transpose(1, 2)
        cos, sin = o.rope_cos_sin(m.rope.inv_freq(), torch.arange(P))
        q = o.apply_rope(q, cos.double(), sin.double())
        core = o.prefill_attention(q, [bk[h] for h in range(Hkv)], [torch.from_numpy(kx[:, h]).double() for h in range(Hkv)],
                                   torch.from_numpy(vx).double(), m.v_proj.U.weight.double().cpu(), cos.double(),
                                   sin.double(), kv_dtype=torch.float16)
        ref = core.transpose(1, 2).reshape(B, P, -1) @ m.o_proj.weight.double().cpu().T
        check_output(pre, ref, f"prefill P={P} (o_proj output): ")
        for t in range(P, P + 3):
            pos = torch.full((B, 1), t, device="cuda")
            out, _ = m(hid[:, t:t + 1], rot(hid[:, t:t + 1], pos), None, pos, *caches)
            torch.cuda.synchronize()
            # fp64 attention over the module's own (dequantised) caches
            kx, vx = dequantised()
            S = kx.shape[2]
            q = (hid[:, t:t + 1].double().cpu() @ m.q_proj.weight.double().cpu().T).view(B, 1, Hq, HEAD).transpose(1, 2)
            cos, sin = o.rope_cos_sin(m.rope.inv_freq(), torch.arange(t, t + 1))
            q = o.apply_rope(q[:, :, 0], cos.double(), sin.double())
            cos, sin = o.rope_cos_sin(m.rope.inv_freq(), torch.arange(S))
            core, _, _ = o.decode_attention(q, [bk[h] for h in range(Hkv)], [torch.from_numpy(kx[:, h]).double() for h in range(Hkv)],
                                            torch.from_numpy(vx).double(), m.v_proj.U.weight.double().cpu(), cos.double(), sin.double())
            ref = core.reshape(B, 1, -1) @ m.o_proj.weight.double().cpu().T
            # o_proj is linear: the core's gates carry over to its output (the
            # fp16 projection rounds at 2^-11, well inside them)
            check_output(out, ref, f"decode t={t} S={S} (o_proj output): ")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["dense", "int8_g64"])
def test_k_append_packed_heads_equals_padded_layout(fmt):
    """The K writer fed the latent projection's packed rows [B, T, sum(r)]
    (per-head source offsets) stores exactly what it stores from the padded
    [B, Hkv, T, r_max] layout."""
    from starkv.cache import LatentCache
    print(f"[cache] packed K source fmt={fmt}", flush=True)
    ranks, Rv, B, T = [24, 8, 40, 16], 64, 2, 19
    g = torch.Generator(device="cuda").manual_seed(12)
    packed = torch.randn(B, T, sum(ranks), generator=g, device="cuda").half()
    padded = torch.zeros(B, len(ranks), T, max(ranks), device="cuda", dtype=torch.float16)
    off = 0
    for h, r in enumerate(ranks):
        padded[:, h, :, :r] = packed[:, :, off:off + r]
        off += r
    v_new = torch.randn(B, T, Rv, generator=g, device="cuda").half()
    bk = torch.zeros(len(ranks), max(ranks), 128, device="cuda", dtype=torch.float16)
    caches = []
    for src in (padded, packed):
        c = LatentCache(B, ranks, Rv, T + 5, torch.float16, "cuda", fmt=fmt)
        c.append(src[:, :, :7] if src.dim() == 4 else src[:, :7], v_new[:, :7], bk)
        c.append(src[:, :, 7:] if src.dim() == 4 else src[:, 7:], v_new[:, 7:], bk)
        caches.append(c)
    torch.cuda.synchronize()
    assert torch.equal(caches[0].k_data, caches[1].k_data)
    if fmt != "dense":
        assert torch.equal(caches[0].k_scale, caches[1].k_scale)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["dense", "int8_g64", "reference"])
@pytest.mark.parametrize("device_pos", [False, True])
def test_decode_append_equals_the_three_writes(fmt, device_pos):
    """starkv_decode_append (K write, V write and query rotation in one launch)
    stores exactly what starkv_k_append, starkv_v_append and starkv_rope_apply
    store one by one, for each cache format, at a host or a device position."""
    from starkv import RopeConfig
    from starkv.cache import LatentCache
    from starkv.ops import k_append, rope_apply, v_append
    print(f"[cache] decode_append fmt={fmt} device_pos={device_pos}", flush=True)
    ranks, Rv, B, T, cap, pos = [24, 8, 40, 16], 264, 2, 3, 32, 9
    g = torch.Generator(device="cuda").manual_seed(17)
    k_new = torch.randn(B, T, sum(ranks), generator=g, device="cuda").half()
    v_new = torch.randn(B, T, Rv, generator=g, device="cuda").half()
    bk = torch.randn(len(ranks), max(ranks), HEAD, generator=g, device="cuda").half()
    q0 = torch.randn(B, 8, T, HEAD, generator=g, device="cuda").half()
    rope = RopeConfig(theta=500000.0)
    a, b = (LatentCache(B, ranks, Rv, cap, torch.float16, "cuda", fmt=fmt) for _ in range(2))
    qa, qb = q0.clone(), q0.clone()
    if device_pos:
        p = torch.tensor([pos], dtype=torch.int32, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        a.append_at(k_new, v_new, bk, p, error_flag=err, q=qa, rope=rope)
        ks = b.k_spec(bk)
        k_append(k_new, ks, 0, cap, pos0_device=p, error_flag=err)
        v_append(v_new, b.v_spec, 0, cap, pos0_device=p, error_flag=err)
        rope_apply(qb, rope, pos0_device=p, max_positions=cap, error_flag=err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
    else:
        a.length = b.length = pos
        a.append(k_new, v_new, bk, q=qa, rope=rope)
        ks = b.k_spec(bk)
        k_append(k_new, ks, pos, cap)
        v_append(v_new, b.v_spec, pos, cap)
        rope_apply(qb, rope, pos0=pos)
        torch.cuda.synchronize()
    assert torch.equal(qa, qb) and not torch.equal(qa, q0)
    for name in ("k_data", "k_scale", "k_data2", "k_scale2", "v_data", "v_scale", "v_zero", "v_data2", "v_scale2"):
        ta, tb = getattr(a, name, None), getattr(b, name, None)
        if ta is not None:
            assert torch.equal(ta, tb), name
