"""GPU tests of the quantised V-latent formats (P.V kernel, fused decode, bx drop-in).

Quantised caches are written with the oracle's quantisers on the CPU and
uploaded; the expected dequantised values come from the oracle's dequant
functions (numpy, integer-exact, one fp16 rounding; bf16 activations round
that fp16 value once more, as torch_bx's ``.to(b.dtype)`` does).

Bit-exactness of the dequantisation is checked through the kernel with a
one-hot P: every head selects one position, so out[b, h, :] is that
position's dequantised row (exact products by 1.0, fp32 accumulation, exact
output rounding).
"""
import math
import sys

import numpy as np
import pytest
import torch

from _util import errors

HEAD = 128


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev_pitched(a, pad):
    """[B, S, n] bytes on the GPU inside rows of n + pad bytes, starting one
    byte into an allocation: rows of any alignment (a view, as a caller's
    cache slice would be)."""
    if not pad:
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()
    B, S, n = a.shape
    big = torch.zeros(B, S, n + pad + 1, dtype=torch.from_numpy(a[:0]).dtype, device="cuda")
    v = big[..., 1:1 + n]
    v.copy_(torch.from_numpy(np.ascontiguousarray(a)).cuda())
    return v


def make_quant_v(kind, B, S, R, split=256, seed=0, outliers=True, pad=0):
    """Returns (VLatentSpec on cuda, dequantised V as fp16 numpy [B, S, R], float V).
    pad > 0: the packed rows sit unaligned (one byte in, pitch + pad)."""
    from oracle import starkv_oracle as o
    from starkv import VLatentSpec
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, S, R)).astype(np.float32)
    if outliers:
        x[..., ::97] *= 10.0                                           # 1 % outlier channels
    dev = lambda a: (_dev_pitched(a, pad) if a.dtype in (np.uint8, np.int8)
                     else torch.from_numpy(np.ascontiguousarray(a)).cuda())
    if kind in ("ref_int4", "ref_int8"):
        lo_r = R - split
        if kind == "ref_int4":
            p1, s1 = o.quant_int4_ref(x[..., :split])
            d1 = o.dequant_int4_ref(p1, s1, split)
            x1 = dev(p1)
        else:
            q1, s1 = o.quant_int8_sym(x[..., :split])
            d1 = o.dequant_int8_sym(q1, s1)
            x1 = dev(q1)
        p2, s2 = o.quant_int4_ref(x[..., split:])
        d2 = o.dequant_int4_ref(p2, s2, lo_r)
        spec = VLatentSpec.int4_ref(x1, dev(s1), R, split=split, x2=dev(p2), scale2=dev(s2))
        return spec, np.concatenate([d1, d2], axis=-1), x
    if kind == "int4_whole":
        p, s = o.quant_int4_ref(x)
        return VLatentSpec.int4_ref(dev(p), dev(s), R), o.dequant_int4_ref(p, s, R), x
    if kind == "int8":
        q, s = o.quant_int8_sym(x)
        return VLatentSpec.int8(dev(q), dev(s)), o.dequant_int8_sym(q, s), x
    if kind == "g64":
        n, sc, zr = o.quant_int4_asym(x, 64)
        packed = o.pack_int4_ref(n.astype(np.int16) - 8)                 # unsigned nibbles n
        return VLatentSpec.int4_g64(dev(packed), dev(sc), dev(zr), R), o.dequant_int4_asym(n, sc, zr, 64), x
    raise ValueError(kind)


KINDS = [("ref_int4", 384, 256), ("ref_int8", 1640, 256), ("int4_whole", 512, 512), ("int8", 264, 264),
         ("g64", 1640, 0), ("g64", 200, 0)]
# ranks that are not multiples of 8 (rows of any byte length: the reference's
# bx default R = 1228 over 256 upper ranks leaves 486-byte lower rows), and
# aligned ranks in rows placed one byte into their buffer (pad)
ODD_KINDS = [("ref_int4", 1228, 256, 0), ("ref_int8", 1228, 256, 0), ("ref_int4", 1227, 256, 0),
             ("int4_whole", 203, 203, 0), ("int8", 77, 77, 0), ("g64", 203, 0, 0), ("g64", 1229, 0, 0),
             ("ref_int4", 384, 256, 3), ("int8", 264, 264, 5), ("g64", 1640, 0, 2)]


def _dequant_one_hot(kind, R, split, dtype, pad=0):
    from starkv import pv_latent
    B, S, H = 2, 45, 32
    spec, deq, _ = make_quant_v(kind, B, S, R, split=split or 256, seed=R, pad=pad)
    p = torch.zeros(B, H, S, dtype=dtype, device="cuda")
    pick = [[(7 * h + 3 * b) % S for h in range(H)] for b in range(B)]
    for b in range(B):
        for h in range(H):
            p[b, h, pick[b][h]] = 1.0
    out = pv_latent(p, spec)
    torch.cuda.synchronize()
    want = torch.from_numpy(np.stack([deq[b][pick[b]] for b in range(B)])).to(dtype)
    got = out.cpu()
    bad = (got.view(torch.int16) != want.view(torch.int16)).sum().item()
    _flush(f"   mismatching values: {bad} of {got.numel()}")
    assert bad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kind,R,split", KINDS)
def test_pv_dequant_bit_exact(kind, R, split, dtype):
    _flush(f"[dequant] {kind} R={R} split={split} {dtype}")
    _dequant_one_hot(kind, R, split, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kind,R,split,pad", ODD_KINDS)
def test_pv_dequant_bit_exact_any_rank(kind, R, split, pad, dtype):
    _flush(f"[dequant any rank] {kind} R={R} split={split} pad={pad} {dtype}")
    _dequant_one_hot(kind, R, split, dtype, pad=pad)


@pytest.mark.gpu
@pytest.mark.parametrize("kind,R,split", [KINDS[0], KINDS[1], KINDS[4]])
def test_pv_quant_matches_oracle(kind, R, split):
    from starkv import pv_latent
    _flush(f"[pv quant] {kind} R={R}")
    B, S, H = 3, 700, 32
    spec, deq, _ = make_quant_v(kind, B, S, R, split=split or 256, seed=1)
    g = torch.Generator(device="cuda").manual_seed(2)
    p = torch.softmax(torch.randn(B, H, S, generator=g, device="cuda") * 3, dim=-1).half()
    out = pv_latent(p, spec)
    ref = p.double().cpu() @ torch.from_numpy(deq).double()
    mx, mr = errors(out.float(), ref)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mr <= 1e-3 and mx <= 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("kind,R,split", [("ref_int4", 1640, 256), ("g64", 1640, 0)])
def test_decode_with_quantised_v(kind, R, split):
    from oracle import starkv_oracle as o
    from starkv import RopeConfig, decode_attention
    from _util import make_case
    _flush(f"[decode quant v] {kind} R={R}")
    B, H, S = 2, 32, 1000
    ranks = [32, 48, 64, 16] * 8
    case = make_case(B, H, H, S, ranks, R, dtype=torch.float16, seed=3)
    spec, deq, _ = make_quant_v(kind, B, S, R, split=split or 256, seed=4)
    out = decode_attention(case.q, case.kspec, spec, case.uv, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rope = RopeConfig()
    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)
    ref, _, _ = o.decode_attention(case.q.cpu(), [b.cpu() for b in case.bk_heads], [x.cpu() for x in case.xk_heads],
                                   torch.from_numpy(deq), case.uv.cpu(), cos, sin)
    mx, mr = errors(out, ref)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mr <= 1e-3 and mx <= 2e-2


# Group-64 V with aligned rows takes the raw-nibble P.V kernel (8 waves over
# 33..64 column tiles, 4 waves up to 16 tiles): both activation dtypes, an odd
# tile count, a half last group with two head groups, the largest rank, long
# contexts (many splits), contexts that are not multiples of its 32-position
# step, one partial step, and rows that take its 16-byte copies.
G64_WIDE = [("bf16_1640", torch.bfloat16, 1640, 32, 777), ("f16_1056_odd_tiles", torch.float16, 1056, 32, 650),
            ("f16_1096_half_group_h64", torch.float16, 1096, 64, 1500), ("f16_2048", torch.float16, 2048, 32, 333),
            ("bf16_1288_long", torch.bfloat16, 1288, 32, 6001), ("f16_1640_s5", torch.float16, 1640, 32, 5),
            # rows of whole 16-byte pieces (640 and 528 bytes): 16-byte copies
            ("bf16_1280_d16", torch.bfloat16, 1280, 32, 1111),
            # up to 16 tiles: the 4-wave shape (one or two groups per wave)
            ("bf16_512_s33", torch.bfloat16, 512, 32, 33), ("f16_480_h64", torch.float16, 480, 64, 2100),
            ("f16_256_s1", torch.float16, 256, 32, 1),
            ("bf16_136_long", torch.bfloat16, 136, 32, 9000)]


@pytest.mark.gpu
@pytest.mark.parametrize("name,dtype,R,H,S", G64_WIDE, ids=[c[0] for c in G64_WIDE])
def test_decode_g64_all_columns(name, dtype, R, H, S):
    from oracle import starkv_oracle as o
    from starkv import RopeConfig, decode_attention
    from _util import make_case
    _flush(f"[decode g64 all columns] {name}: R={R} H={H} S={S} {dtype}")
    B = 2
    case = make_case(B, H, H, S, [32, 48, 64, 16] * (H // 4), R, dtype=dtype, seed=R + S)
    spec, deq, _ = make_quant_v("g64", B, S, R, seed=S)
    out = decode_attention(case.q, case.kspec, spec, case.uv, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rope = RopeConfig()
    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)
    v = torch.from_numpy(deq)
    if dtype == torch.bfloat16:
        v = v.to(torch.bfloat16)                     # the P.V operand, as torch_bx's .to(b.dtype)
    ref, _, _ = o.decode_attention(case.q.cpu(), [b.cpu() for b in case.bk_heads], [x.cpu() for x in case.xk_heads],
                                   v, case.uv.cpu(), cos, sin)
    mx, mr = errors(out, ref)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mr <= 1e-3 and mx <= 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("R,S", [(1640, 700), (200, 300)])
def test_decode_g64_dequant_bit_exact(R, S, dtype):
    """The fused decode's dequantisation, exactly: a mask that leaves one
    position per (batch, head) makes P one-hot (exp(0) = 1, sum 1), and a
    one-hot U_v picks 128 V ranks per head, so every fp32 output is one
    dequantised value fp16(n * s + z) (bf16 models: rounded once more to
    bf16), bit for bit.  R = 1640 runs the all-columns raw-nibble P.V kernel,
    R = 200 the column-block kernel."""
    from starkv import decode_attention
    from _util import make_case
    _flush(f"[decode g64 bit-exact] R={R} S={S} {dtype}")
    B, H = 2, 32
    case = make_case(B, H, H, S, [32, 48, 64, 16] * 8, R, dtype=dtype, seed=R)
    spec, deq, _ = make_quant_v("g64", B, S, R, seed=R + 1)
    pick = [[(37 * h + 11 * b + 5) % S for h in range(H)] for b in range(B)]
    mask = torch.full((B, H, S), -1e30, dtype=torch.float32, device="cuda")
    for b in range(B):
        for h in range(H):
            mask[b, h, pick[b][h]] = 0.0
    sel = torch.tensor([[(97 * h + 13 * d) % R for d in range(HEAD)] for h in range(H)])
    uv = torch.zeros(H * HEAD, R, dtype=dtype)
    uv[torch.arange(H * HEAD), sel.reshape(-1)] = 1.0
    out = decode_attention(case.q, case.kspec, spec, uv.cuda(), mask=mask, out_dtype=torch.float32)
    torch.cuda.synchronize()
    v = torch.from_numpy(deq)
    if dtype == torch.bfloat16:
        v = v.to(torch.bfloat16)
    want = torch.stack([torch.stack([v[b, pick[b][h]][sel[h]] for h in range(H)]) for b in range(B)]).float()
    bad = (out.cpu() != want).sum().item()
    _flush(f"   mismatching values: {bad} of {want.numel()}")
    assert bad == 0


@pytest.mark.gpu
@pytest.mark.parametrize("upper", ["int4", "int8"])
def test_bx_dropin(upper):
    from oracle import starkv_oracle as o
    from starkv.bx_quant import bx
    _flush(f"[bx] upper={upper}")
    B, S, H, R, U = 2, 333, 32, 1024, 256
    rng = np.random.default_rng(9)
    x = rng.standard_normal((B, S, R)).astype(np.float32)
    if upper == "int4":
        p1, s1 = o.quant_int4_ref(x[..., :U])
        d1 = o.dequant_int4_ref(p1, s1, U)
    else:
        p1, s1 = o.quant_int8_sym(x[..., :U])
        d1 = o.dequant_int8_sym(p1, s1)
    p2, s2 = o.quant_int4_ref(x[..., U:])
    deq = np.concatenate([d1, o.dequant_int4_ref(p2, s2, R - U)], axis=-1)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    g = torch.Generator(device="cuda").manual_seed(10)
    p = torch.softmax(torch.randn(B, H, S, generator=g, device="cuda"), dim=-1).half()
    out = bx(p, dev(p1), dev(p2), dev(s1), dev(s2), original_rank=R, upper_rank=U)
    assert out.shape == (B, H, R) and out.dtype == torch.float16
    ref = p.double().cpu() @ torch.from_numpy(deq).double()
    mx, mr = errors(out.float(), ref)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mr <= 1e-3 and mx <= 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("upper", ["int4", "int8"])
def test_bx_reference_check_shape(upper):
    """The reference's own bx check (bx_quant.py:224-248, defaults 245-252):
    B 16, 32 heads, S 4096, total rank int(0.3 * 4096) = 1228 over 256 upper
    ranks (a 972-rank lower block: 486-byte int4 rows), fp16, P ~ N(0, 1).
    The dequantisation is bit-exact (one-hot P over the first batches) and the
    output meets the attention gate against the oracle in float64."""
    from oracle import starkv_oracle as o
    from starkv.bx_quant import bx
    B, H, S, R, U = 16, 32, 4096, int(0.3 * 4096), 256
    _flush(f"[bx reference shape] B={B} S={S} R={R} upper={U} ({upper})")
    rng = np.random.default_rng(11)
    x = rng.standard_normal((B, S, R)).astype(np.float32)
    x[..., ::97] *= 10.0
    if upper == "int4":
        p1, s1 = o.quant_int4_ref(x[..., :U])
        d1 = o.dequant_int4_ref(p1, s1, U)
    else:
        p1, s1 = o.quant_int8_sym(x[..., :U])
        d1 = o.dequant_int8_sym(p1, s1)
    p2, s2 = o.quant_int4_ref(x[..., U:])
    assert p2.shape[-1] == 486
    deq = np.concatenate([d1, o.dequant_int4_ref(p2, s2, R - U)], axis=-1)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    x1, x2, sc1, sc2 = dev(p1), dev(p2), dev(s1), dev(s2)
    # one-hot P: each head of batches 0..1 picks one position -> its dequantised row
    p = torch.zeros(B, H, S, dtype=torch.float16, device="cuda")
    pick = [[(131 * h + 17 * b) % S for h in range(H)] for b in range(2)]
    for b in range(2):
        for h in range(H):
            p[b, h, pick[b][h]] = 1.0
    out = bx(p, x1, x2, sc1, sc2, original_rank=R, upper_rank=U)
    torch.cuda.synchronize()
    want = torch.from_numpy(np.stack([deq[b][pick[b]] for b in range(2)])).half()
    got = out[:2].cpu()
    bad = (got.view(torch.int16) != want.view(torch.int16)).sum().item()
    _flush(f"   one-hot mismatching values: {bad} of {got.numel()}")
    assert bad == 0
    assert torch.count_nonzero(out[2:]).item() == 0
    # the reference's own probabilities: N(0, 1), fp16
    g = torch.Generator(device="cuda").manual_seed(12)
    p = torch.randn(B, H, S, generator=g, device="cuda").half()
    out = bx(p, x1, x2, sc1, sc2, original_rank=R, upper_rank=U)
    torch.cuda.synchronize()
    assert out.shape == (B, H, R) and out.dtype == torch.float16
    ref = p.double().cpu() @ torch.from_numpy(deq).double()
    mx, mr = errors(out.float(), ref)
    # P is not normalised here, so |out| reaches ~1e2: the max-abs gate of 2e-2
    # applies per element to max(1, |ref|) (an fp16 output keeps ~5e-4 relative)
    scaled = ((out.double().cpu() - ref).abs() / ref.abs().clamp_min(1.0)).max().item()
    _flush(f"   max_abs={mx:.3e} scaled max_abs={scaled:.3e} mean_rel={mr:.3e}  (|ref| mean {ref.abs().mean():.2f})")
    assert mr <= 1e-3 and scaled <= 2e-2
