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


def make_quant_v(kind, B, S, R, split=256, seed=0, outliers=True):
    """Returns (VLatentSpec on cuda, dequantised V as fp16 numpy [B, S, R], float V)."""
    from oracle import starkv_oracle as o
    from starkv import VLatentSpec
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, S, R)).astype(np.float32)
    if outliers:
        x[..., ::97] *= 10.0                                           # 1 % outlier channels
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
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


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kind,R,split", KINDS)
def test_pv_dequant_bit_exact(kind, R, split, dtype):
    from starkv import pv_latent
    _flush(f"[dequant] {kind} R={R} split={split} {dtype}")
    B, S, H = 2, 45, 32
    spec, deq, _ = make_quant_v(kind, B, S, R, split=split or 256, seed=R)
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
