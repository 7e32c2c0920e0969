"""GPU tests of the quantised K-latent formats (K-logit kernel, fused decode, quant abx drop-in).

Caches are quantised with the oracle's quantisers on the CPU; the oracle
computes the logits / attention from the oracle-dequantised (fp16) latents,
which is what the kernel uses after its bit-exact dequantisation.
"""
import math
import sys

import numpy as np
import pytest
import torch

from _util import cfg2_ranks, check_logits, check_output, errors

HEAD = 128


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _rope_cs(S, rope=None):
    from oracle import starkv_oracle as o
    from starkv import RopeConfig
    rope = rope or RopeConfig()
    return o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)


def ragged_int8_k(B, S, ranks, seed=0):
    """int8 K latent with one fp16 scale per (b, h, s), heads back to back per
    batch ([S, r_h] bytes each).  Returns (KLatentSpec pieces, dequantised
    per-head [B, S, r_h] float64 tensors)."""
    from oracle import starkv_oracle as o
    rng = np.random.default_rng(seed)
    Hkv = len(ranks)
    per_b = S * sum(ranks)
    buf = np.zeros((B, per_b), np.int8)
    scales = np.zeros((B, Hkv, S), np.float16)
    deq, offs = [], []
    off = 0
    for h, r in enumerate(ranks):
        x = rng.standard_normal((B, S, r)).astype(np.float32)
        x[..., ::13] *= 8.0
        q, s = o.quant_int8_sym(x)
        buf[:, off:off + S * r] = q.reshape(B, S * r)
        scales[:, h, :] = s[..., 0]
        deq.append(torch.from_numpy(o.dequant_int8_sym(q, s).astype(np.float64)))
        offs.append(off)
        off += S * r
    return buf, scales, offs, deq


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,S", [(2, 700),
                                 (1, 31), (1, 64),      # one and two tiles: the pipelined int8 loop's edges
                                 (1, 4099), (4, 2100)])  # chunks of many tiles, partial last tile
def test_k_logits_int8_ragged(dtype, B, S):
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, k_logits
    from starkv._lib import FMT_INT8_SYM
    _flush(f"[k int8 ragged] {dtype} B={B} S={S}")
    ranks = cfg2_ranks()
    Hkv = len(ranks)
    buf, scales, offs, deq = ragged_int8_k(B, S, ranks, seed=1)
    g = torch.Generator(device="cuda").manual_seed(2)
    q = torch.randn(B, Hkv, HEAD, generator=g, device="cuda").to(dtype)
    bk_all = torch.randn(sum(ranks), HEAD, generator=g, device="cuda")
    bko = list(np.cumsum([0] + ranks[:-1]) * HEAD)
    for h, r in enumerate(ranks):
        bk_all[bko[h] // HEAD:bko[h] // HEAD + r] /= math.sqrt(r)
    bk_all = bk_all.to(dtype)
    sc = _dev(scales)
    spec = KLatentSpec(_dev(buf), ranks, offs, ranks, buf.shape[1], bk_all, bko, HEAD,
                       fmt=FMT_INT8_SYM, scale=sc, scale_stride_b=sc.stride(0), scale_stride_h=sc.stride(1))
    out = k_logits(q, spec, S, scale=0.5)
    torch.cuda.synchronize()
    cos, sin = _rope_cs(S)
    bk_h = [bk_all[bko[h] // HEAD:bko[h] // HEAD + r].cpu() for h, r in enumerate(ranks)]
    ref = o.k_logits(q.cpu(), bk_h, deq, cos, sin, scale=0.5)
    check_logits(out, ref, 0.5)


@pytest.mark.gpu
@pytest.mark.parametrize("S,scale_pitch,gqa", [(700, 704, False),   # staged scales, last piece past S
                                                (700, 700, False),   # pitch < round_up(S, 8): other kernel
                                                (1000, 1000, False),
                                                (333, 336, True)])
def test_k_logits_int8_padded_rows(S, scale_pitch, gqa):
    """int8 K with rows padded to 16 bytes (the cache's layout): the
    warp-specialised kernel stages each tile's scales with its rows when the
    scale rows are readable through round_up(S, 8)."""
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, k_logits
    from starkv._lib import FMT_INT8_SYM
    _flush(f"[k int8 padded] S={S} scale_pitch={scale_pitch} gqa={gqa}")
    B = 3
    ranks = [32, 48, 16, 64, 32, 56, 16, 96] if gqa else cfg2_ranks()
    Hkv = len(ranks)
    Hq = 4 * Hkv if gqa else Hkv
    pitch = [(r + 15) // 16 * 16 for r in ranks]
    rng = np.random.default_rng(S)
    buf = np.zeros((B, S * sum(pitch)), np.int8)
    scales = np.zeros((B, Hkv, scale_pitch), np.float16)
    scales[..., S:] = np.float16(np.inf)        # never used: positions past S
    deq, offs, off = [], [], 0
    for h, r in enumerate(ranks):
        x = rng.standard_normal((B, S, r)).astype(np.float32)
        x[..., ::13] *= 8.0
        q, s = o.quant_int8_sym(x)
        rows = np.zeros((B, S, pitch[h]), np.int8)
        rows[..., :r] = q
        buf[:, off:off + S * pitch[h]] = rows.reshape(B, -1)
        scales[:, h, :S] = s[..., 0]
        deq.append(torch.from_numpy(o.dequant_int8_sym(q, s).astype(np.float64)))
        offs.append(off)
        off += S * pitch[h]
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn(B, Hq, HEAD, generator=g, device="cuda").half()
    bko = list(np.cumsum([0] + ranks[:-1]) * HEAD)
    bk_all = torch.cat([torch.randn(r, HEAD, generator=g, device="cuda") / math.sqrt(r) for r in ranks]).half()
    sc = _dev(scales)
    spec = KLatentSpec(_dev(buf), ranks, offs, pitch, buf.shape[1], bk_all, bko, HEAD,
                       fmt=FMT_INT8_SYM, scale=sc, scale_stride_b=sc.stride(0), scale_stride_h=sc.stride(1))
    out = k_logits(q, spec, S, scale=0.25)
    torch.cuda.synchronize()
    cos, sin = _rope_cs(S)
    bk_h = [bk_all[bko[h] // HEAD:bko[h] // HEAD + r].cpu() for h, r in enumerate(ranks)]
    ref = o.k_logits(q.cpu(), bk_h, deq, cos, sin, scale=0.25)
    check_logits(out, ref, 0.25)


def reference_split_k(B, H, S, upper, lower, upper_kind="int8", seed=0):
    """The reference module's split K cache [B, H, S, *] and its dequantised [B, H, S, upper+lower]."""
    from oracle import starkv_oracle as o
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, H, S, upper + lower)).astype(np.float32)
    if upper_kind == "int8":
        q1, s1 = o.quant_int8_sym(x[..., :upper])
        d1 = o.dequant_int8_sym(q1, s1)
    else:
        q1, s1 = o.quant_int4_ref(x[..., :upper])
        d1 = o.dequant_int4_ref(q1, s1, upper)
    parts = [d1]
    q2 = s2 = None
    if lower:
        q2, s2 = o.quant_int4_ref(x[..., upper:])
        parts.append(o.dequant_int4_ref(q2, s2, lower))
    return q1, s1, q2, s2, np.concatenate(parts, axis=-1).astype(np.float64)


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,upper,lower,kind,repeat", [
    (32, 32, 16, 48, "int8", False),
    (32, 8, 16, 112, "int8", False),
    (32, 8, 16, 112, "int8", True),      # cache repeated per query head, as the reference module does
    (8, 8, 32, 96, "int4", False),
    (8, 8, 0, 64, "int4", False),        # whole-rank int4
])
def test_k_logits_reference_split(Hq, Hkv, upper, lower, kind, repeat):
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, k_logits
    _flush(f"[k split] Hq={Hq} Hkv={Hkv} upper={upper} lower={lower} {kind} repeat={repeat}")
    B, S = 2, 513
    r = upper + lower
    if upper == 0:
        q1, s1, _, _, deq = reference_split_k(B, Hkv, S, lower, 0, "int4", seed=3)
    else:
        q1, s1, q2, s2, deq = reference_split_k(B, Hkv, S, upper, lower, kind, seed=3)
    g = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn(B, Hq, HEAD, generator=g, device="cuda").half()
    bk = (torch.randn(Hkv, r, HEAD, generator=g, device="cuda") / math.sqrt(r)).half()
    rep = (lambda a: np.repeat(a, Hq // Hkv, axis=1)) if repeat else (lambda a: a)
    if upper == 0:
        spec = KLatentSpec.from_reference_quant(_dev(rep(q1)), _dev(rep(s1)), bk, r)
    else:
        spec = KLatentSpec.from_reference_quant(_dev(rep(q1)), _dev(rep(s1)), bk, r, x2=_dev(rep(q2)),
                                                s2=_dev(rep(s2)), split=upper)
    out = k_logits(q, spec, S)
    torch.cuda.synchronize()
    cos, sin = _rope_cs(S)
    ref = o.k_logits(q.cpu(), [bk[h].cpu() for h in range(Hkv)], [torch.from_numpy(deq[:, h]) for h in range(Hkv)],
                     cos, sin)
    check_logits(out, ref, 1.0)


@pytest.mark.gpu
def test_quant_abx_dropin():
    from oracle import starkv_oracle as o
    from starkv.abx_rope_batched_quant import abx
    _flush("[quant abx] Hq=32 Hkv=8 upper 16 int8 + lower 112 int4, cache repeated per query head")
    B, Hq, Hkv, S, U, L = 2, 32, 8, 300, 16, 112
    q1, s1, q2, s2, deq = reference_split_k(B, Hkv, S, U, L, "int8", seed=5)
    g = torch.Generator(device="cuda").manual_seed(6)
    A = torch.randn(B, Hq, 1, HEAD, generator=g, device="cuda").half()
    Bk = (torch.randn(Hkv, U + L, HEAD, generator=g, device="cuda") / math.sqrt(U + L)).half()
    rep = lambda a: np.repeat(a, Hq // Hkv, axis=1)
    out = abx(A, Bk, _dev(rep(q1)), _dev(rep(q2)), _dev(rep(s1)), _dev(rep(s2)), L)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, 1, S) and out.dtype == torch.float16
    cos, sin = _rope_cs(S)
    ref = o.k_logits(A[:, :, 0].cpu(), [Bk[h].cpu() for h in range(Hkv)], [torch.from_numpy(deq[:, h]) for h in range(Hkv)],
                     cos, sin)
    check_logits(out[:, :, 0], ref, 1.0)      # fp16 logits, as the reference abx returns


@pytest.mark.gpu
def test_decode_int8_k_g64_v():
    """cfg3's formats (int8 K per (b, h, s); int4 group-64 V) through the fused decode."""
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, decode_attention
    from starkv._lib import FMT_INT8_SYM
    from test_gpu_quant import make_quant_v
    _flush("[decode int8 K + g64 V] ragged cfg2 ranks, Rv 1640")
    B, S, Rv = 2, 900, 1640
    ranks = cfg2_ranks()
    Hkv = len(ranks)
    buf, scales, offs, deq_k = ragged_int8_k(B, S, ranks, seed=7)
    vspec, deq_v, _ = make_quant_v("g64", B, S, Rv, seed=8)
    g = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(B, Hkv, HEAD, generator=g, device="cuda").half()
    bko = list(np.cumsum([0] + ranks[:-1]) * HEAD)
    bk_all = torch.cat([torch.randn(r, HEAD, generator=g, device="cuda") / math.sqrt(r) for r in ranks]).half()
    uv = (torch.randn(Hkv * HEAD, Rv, generator=g, device="cuda") / math.sqrt(Rv)).half()
    sc = _dev(scales)
    kspec = KLatentSpec(_dev(buf), ranks, offs, ranks, buf.shape[1], bk_all, bko, HEAD,
                        fmt=FMT_INT8_SYM, scale=sc, scale_stride_b=sc.stride(0), scale_stride_h=sc.stride(1))
    out = decode_attention(q, kspec, vspec, uv, out_dtype=torch.float32)
    torch.cuda.synchronize()
    cos, sin = _rope_cs(S)
    bk_h = [bk_all[bko[h] // HEAD:bko[h] // HEAD + r].cpu() for h, r in enumerate(ranks)]
    ref, _, _ = o.decode_attention(q.cpu(), bk_h, deq_k, torch.from_numpy(deq_v), uv.cpu(), cos, sin)
    check_output(out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_k_logits_int8_any_rank(dtype):
    """int8 K of ranks that are not multiples of 8, heads back to back (rows of
    any byte alignment; the bytes past a row are the next row's): the
    register-streaming kernel's unaligned-row loads, with the ranks past each
    head's rank masked."""
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, k_logits
    from starkv._lib import FMT_INT8_SYM
    ranks = [37, 100, 5, 64, 17, 128, 90, 1, 33, 71, 16, 127]
    _flush(f"[k int8 any rank] ranks {ranks} {dtype}")
    B, S = 2, 517
    Hkv = len(ranks)
    buf, scales, offs, deq = ragged_int8_k(B, S, ranks, seed=21)
    g = torch.Generator(device="cuda").manual_seed(22)
    q = torch.randn(B, Hkv, HEAD, generator=g, device="cuda").to(dtype)
    bko = list(np.cumsum([0] + ranks[:-1]) * HEAD)
    bk_all = torch.cat([torch.randn(r, HEAD, generator=g, device="cuda") / math.sqrt(r) for r in ranks]).to(dtype)
    sc = _dev(scales)
    spec = KLatentSpec(_dev(buf), ranks, offs, ranks, buf.shape[1], bk_all, bko, HEAD,
                       fmt=FMT_INT8_SYM, scale=sc, scale_stride_b=sc.stride(0), scale_stride_h=sc.stride(1))
    out = k_logits(q, spec, S, scale=0.5)
    torch.cuda.synchronize()
    cos, sin = _rope_cs(S)
    bk_h = [bk_all[bko[h] // HEAD:bko[h] // HEAD + r].cpu() for h, r in enumerate(ranks)]
    ref = o.k_logits(q.cpu(), bk_h, deq, cos, sin, scale=0.5)
    check_logits(out, ref, 0.5)


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,upper,lower,kind", [
    (32, 8, 16, 84, "int8"),     # the reference module's K at rank 100 (16 int8 + 84 int4)
    (8, 8, 16, 37, "int8"),      # odd lower block: 19-byte rows
    (8, 4, 32, 21, "int4"),
    (8, 8, 0, 75, "int4"),       # whole-rank int4, 38-byte rows
])
def test_k_logits_reference_split_any_rank(Hq, Hkv, upper, lower, kind):
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, k_logits
    _flush(f"[k split any rank] Hq={Hq} Hkv={Hkv} upper={upper} lower={lower} {kind}")
    B, S = 2, 301
    r = upper + lower
    if upper == 0:
        q1, s1, _, _, deq = reference_split_k(B, Hkv, S, lower, 0, "int4", seed=23)
    else:
        q1, s1, q2, s2, deq = reference_split_k(B, Hkv, S, upper, lower, kind, seed=23)
    g = torch.Generator(device="cuda").manual_seed(24)
    q = torch.randn(B, Hq, HEAD, generator=g, device="cuda").half()
    bk = (torch.randn(Hkv, r, HEAD, generator=g, device="cuda") / math.sqrt(r)).half()
    if upper == 0:
        spec = KLatentSpec.from_reference_quant(_dev(q1), _dev(s1), bk, r)
    else:
        spec = KLatentSpec.from_reference_quant(_dev(q1), _dev(s1), bk, r, x2=_dev(q2), s2=_dev(s2), split=upper)
    out = k_logits(q, spec, S)
    torch.cuda.synchronize()
    cos, sin = _rope_cs(S)
    ref = o.k_logits(q.cpu(), [bk[h].cpu() for h in range(Hkv)], [torch.from_numpy(deq[:, h]) for h in range(Hkv)],
                     cos, sin)
    check_logits(out, ref, 1.0)


@pytest.mark.gpu
def test_decode_any_rank_int8_k_g64_v():
    """Fused decode over int8 K of odd ranks (unaligned rows) and group-64 V of
    rank 1229 (615-byte rows)."""
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, decode_attention
    from starkv._lib import FMT_INT8_SYM
    from test_gpu_quant import make_quant_v
    ranks = [37, 100, 5, 64, 17, 128, 90, 1]
    B, S, Rv = 2, 777, 1229
    _flush(f"[decode any rank] int8 K ranks {ranks}, g64 V Rv={Rv}")
    Hkv = len(ranks)
    buf, scales, offs, deq_k = ragged_int8_k(B, S, ranks, seed=25)
    vspec, deq_v, _ = make_quant_v("g64", B, S, Rv, seed=26)
    g = torch.Generator(device="cuda").manual_seed(27)
    q = torch.randn(B, 4 * Hkv, HEAD, generator=g, device="cuda").half()
    bko = list(np.cumsum([0] + ranks[:-1]) * HEAD)
    bk_all = torch.cat([torch.randn(r, HEAD, generator=g, device="cuda") / math.sqrt(r) for r in ranks]).half()
    uv = (torch.randn(Hkv * HEAD, Rv, generator=g, device="cuda") / math.sqrt(Rv)).half()
    sc = _dev(scales)
    kspec = KLatentSpec(_dev(buf), ranks, offs, ranks, buf.shape[1], bk_all, bko, HEAD,
                        fmt=FMT_INT8_SYM, scale=sc, scale_stride_b=sc.stride(0), scale_stride_h=sc.stride(1))
    out = decode_attention(q, kspec, vspec, uv, out_dtype=torch.float32)
    torch.cuda.synchronize()
    cos, sin = _rope_cs(S)
    bk_h = [bk_all[bko[h] // HEAD:bko[h] // HEAD + r].cpu() for h, r in enumerate(ranks)]
    ref, _, _ = o.decode_attention(q.cpu(), bk_h, deq_k, torch.from_numpy(deq_v), uv.cpu(), cos, sin)
    check_output(out, ref)
