"""GPU parity at the benchmark configurations' full sizes.

* Quantised cache (B16 S32768 and B4 S131072; ragged K ranks summing to
  1640, Rv 1640, fp16): fp16 latents with 1 % outlier channels are written by
  the HIP cache writer (K int8 with one fp16 scale per (b, h, s), V int4
  asymmetric in groups of 64 with fp16 scale and zero); the stored bytes of
  the checked batch equal the oracle's quantisers bit for bit, and the decode
  output over the whole cache matches the fp64 oracle on the oracle-quantised
  history.
* Llama-3.1-8B-shaped GQA (32 query / 8 KV heads, llama3 RoPE with theta
  500000, bf16, B1, ranks per KV head in [32, 128], Rv 512, V int4 g64):
  context sweep 256 .. 131072.

Gates: max-abs 2e-2 and mean-rel 1e-3 against the oracle.
"""
import math
import sys

import numpy as np
import pytest
import torch

from _util import cfg2_ranks, cfg4_ranks, errors, make_case

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_REL = 1e-3
HEAD = 128


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _outliers(n: int, offset: int = 0) -> torch.Tensor:
    """Channel mask with every 97th channel (1 %) set."""
    return ((torch.arange(n) + offset) % 97) == 0


@pytest.mark.parametrize("B,S,check", [(16, 32768, [0, 15]), (4, 131072, [3])])
def test_quantised_cache_full_shape(B, S, check):
    from oracle import starkv_oracle as o
    from starkv import RopeConfig, decode_attention
    from starkv.cache import LatentCache
    _flush(f"[cfg quantised] B={B} S={S} checking batches {check}")
    ranks = cfg2_ranks()
    Hkv = Hq = len(ranks)
    Rv, rmax = 1640, max(ranks)
    g = torch.Generator(device="cuda").manual_seed(0)
    # fp16 latents ~N(0,1) with 1 % of the channels scaled x10
    k_new = torch.randn(B, Hkv, S, rmax, generator=g, device="cuda", dtype=torch.float16)
    offs = np.cumsum([0] + ranks[:-1])
    for h, r in enumerate(ranks):
        m = _outliers(r, int(offs[h])).to("cuda")
        k_new[:, h, :, :r][..., m] *= 10
    v_new = torch.randn(B, S, Rv, generator=g, device="cuda", dtype=torch.float16)
    v_new[..., _outliers(Rv).to("cuda")] *= 10
    bk = torch.zeros(Hkv, rmax, HEAD, device="cuda")
    for h, r in enumerate(ranks):
        bk[h, :r] = torch.randn(r, HEAD, generator=g, device="cuda") / math.sqrt(r)
    bk = bk.half()
    uv = (torch.randn(Hkv * HEAD, Rv, generator=g, device="cuda") / math.sqrt(Rv)).half()
    q = torch.randn(B, Hq, HEAD, generator=g, device="cuda").half()

    cache = LatentCache(B, ranks, Rv, S, torch.float16, "cuda", fmt="int8_g64")
    kspec, vspec, length = cache.append(k_new, v_new, bk)
    assert length == S
    rope = RopeConfig()
    out = decode_attention(q, kspec, vspec, uv, rope=rope, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()

    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)
    G = (Rv + 63) // 64
    for b in check:
        ks = []
        for h, r in enumerate(ranks):
            x = k_new[b, h, :, :r].float().cpu().numpy()
            qk, sk = o.quant_int8_sym(x)
            stored = cache.k_rows(h)[b, :S].cpu().numpy()
            assert np.array_equal(stored, qk), f"K bytes of batch {b} head {h}"
            assert np.array_equal(cache.k_scale[b, h, :S].cpu().numpy().view(np.uint16),
                                  sk[..., 0].view(np.uint16)), f"K scales of batch {b} head {h}"
            ks.append(torch.from_numpy(o.dequant_int8_sym(qk, sk).astype(np.float64))[None])
        xv = v_new[b].float().cpu().numpy()
        n, sc, zr = o.quant_int4_asym(xv, 64)
        packed = o.pack_int4_ref(n.astype(np.int16) - 8)
        assert np.array_equal(cache.v_data[b, :S].cpu().numpy(), packed), f"V bytes of batch {b}"
        assert np.array_equal(cache.v_scale[b, :S].cpu().numpy().view(np.uint16), sc.view(np.uint16))
        assert np.array_equal(cache.v_zero[b, :S].cpu().numpy().view(np.uint16), zr.view(np.uint16))
        assert sc.shape[-1] == G
        v = torch.from_numpy(o.dequant_int4_asym(n, sc, zr, 64).astype(np.float64))[None]
        ref, _, _ = o.decode_attention(q[b:b + 1].cpu(), [bk[h, :r].cpu() for h, r in enumerate(ranks)], ks, v,
                                       uv.cpu(), cos, sin)
        mx, mr = errors(out[b:b + 1], ref)
        _flush(f"   batch {b}: max_abs={mx:.3e} mean_rel={mr:.3e}")
        assert mx <= MAX_ABS and mr <= MEAN_REL, (b, mx, mr)
        del ks, v, ref


@pytest.mark.parametrize("S", [256, 1024, 4096, 16384, 65536, 131072])
def test_llama3_gqa_bf16_int4_v_sweep(S):
    from oracle import starkv_oracle as o
    from starkv import RopeConfig, VLatentSpec, decode_attention
    _flush(f"[cfg gqa llama3] S={S}")
    rope = RopeConfig(theta=500000.0, rope_type="llama3", factor=8.0, low_freq_factor=1.0,
                      high_freq_factor=4.0, original_max_position_embeddings=8192)
    Rv = 512
    case = make_case(1, 32, 8, S, cfg4_ranks(), Rv, dtype=torch.bfloat16, seed=5)
    rng = np.random.default_rng(S)
    xv = rng.standard_normal((1, S, Rv)).astype(np.float32)
    xv[..., ::97] *= 10.0
    n, sc, zr = o.quant_int4_asym(xv, 64)
    packed = o.pack_int4_ref(n.astype(np.int16) - 8)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    vspec = VLatentSpec.int4_g64(dev(packed), dev(sc), dev(zr), Rv)
    out = decode_attention(case.q, case.kspec, vspec, case.uv, rope=rope, out_dtype=torch.float32)
    torch.cuda.synchronize()
    # the kernel multiplies bf16 probabilities with the exact fp16 dequantised
    # values rounded once to bf16 (the MFMA operand type)
    v = torch.from_numpy(o.dequant_int4_asym(n, sc, zr, 64)).to(torch.bfloat16).double()
    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)
    ref, _, _ = o.decode_attention(case.q.cpu(), [x.cpu() for x in case.bk_heads], [x.cpu() for x in case.xk_heads],
                                   v, case.uv.cpu(), cos, sin)
    mx, mr = errors(out, ref)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= MAX_ABS and mr <= MEAN_REL, (mx, mr)


@pytest.mark.parametrize("B,S", [(1, 65536), (2, 20000)])
def test_pv_latent_long_context_split_reduction(B, S):
    """The drop-in P.V at long context and small batch, where the split-S
    partials are summed in two levels."""
    from starkv import pv_latent
    _flush(f"[pv long] B={B} S={S}")
    H, Rv = 32, 512
    g = torch.Generator(device="cuda").manual_seed(7)
    p = torch.softmax(torch.randn(B, H, S, generator=g, device="cuda") * 4, dim=-1).half()
    xv = torch.randn(B, S, Rv, generator=g, device="cuda").half()
    out = pv_latent(p, xv)
    torch.cuda.synchronize()
    ref = p.double().cpu() @ xv.double().cpu()
    mx, mr = errors(out.float(), ref)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= MAX_ABS and mr <= MEAN_REL, (mx, mr)
