"""GPU parity of the fused decode path and the K-logit / P.V entry points
against the CPU oracle (oracle/starkv_oracle.py), same seeded inputs.

Gates: attention outputs within max-abs 2e-2 and
mean-rel 1e-3 of the fp32/fp64 eager oracle."""
import math

import pytest
import torch

from _util import cfg2_ranks, cfg4_ranks, check_logits, errors, make_case, oracle_decode, oracle_logits

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_REL = 1e-3
HEAD_DIM_T = 128


def _flush(msg):
    print(msg, flush=True)


def _run_decode(case, rope=None, mask=None, out_dtype=None):
    from starkv import RopeConfig, decode_attention
    rope = rope or RopeConfig()
    return decode_attention(case.q, case.kspec, case.xv, case.uv, rope=rope, mask=mask, out_dtype=out_dtype)


def _check(case, ref, rope=None, mask=None):
    """fp16 cases gate the stored output; bf16 cases gate the fp32 output
    (bf16 storage alone costs ~1.4e-3 mean-rel) and check the stored bf16
    output against the oracle rounded to bf16."""
    if case.dtype == torch.bfloat16:
        out32 = _run_decode(case, rope, mask, out_dtype=torch.float32)
        outbf = _run_decode(case, rope, mask)
        mx, mr = errors(out32, ref)
        d = (outbf.float().cpu().double() - ref.to(torch.bfloat16).double()).abs()
        mr_bf = float(d.mean() / ref.abs().mean())
        _flush(f"   fp32-out max_abs={mx:.3e} mean_rel={mr:.3e}; bf16-out vs bf16(ref) mean_rel={mr_bf:.3e}")
        assert mr_bf <= MEAN_REL, mr_bf
    else:
        out = _run_decode(case, rope, mask)
        assert torch.isfinite(out).all()
        mx, mr = errors(out, ref)
        _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= MAX_ABS and mr <= MEAN_REL, (mx, mr)


CASES = [
    # name, B, Hq, Hkv, S, ranks, Rv, dtype, layout
    # config 1 (the CPU-baseline layer: B1, 32 x 128, S1024, r32 per head,
    # Rv1024, seeded N(0,1) latents, B_k ~N(0,1/32), B_v ~N(0,1/1024), theta
    # 10000) on the HIP path, its fp32 inputs cast to fp16 and to bf16
    ("cfg1_f16", 1, 32, 32, 1024, [32] * 32, 1024, torch.float16, "reference"),
    ("cfg1_bf16", 1, 32, 32, 1024, [32] * 32, 1024, torch.bfloat16, "reference"),
    ("mha_uniform_ref", 2, 32, 32, 1000, [32] * 32, 256, torch.float16, "reference"),
    ("mha_ragged_cfg2ranks", 2, 32, 32, 777, None, 1640, torch.float16, "ragged"),
    ("gqa4_ragged", 2, 32, 8, 1500, [32, 128, 32, 80, 32, 64, 80, 64], 512, torch.float16, "ragged"),
    ("bf16_ragged", 2, 32, 32, 600, None, 1640, torch.bfloat16, "ragged"),
    ("s1", 3, 32, 32, 1, [16] * 32, 64, torch.float16, "reference"),
    ("s33_rv40", 1, 32, 32, 33, [24] * 32, 40, torch.float16, "reference"),
    ("unaligned_r_rv", 2, 32, 32, 129, [20] * 32, 50, torch.float16, "reference"),
    ("mqa_hq8", 2, 8, 1, 300, [128], 128, torch.float16, "ragged"),
    # V wider than one P.V workgroup's 52 column tiles: several column blocks
    ("rv2048_two_blocks", 2, 32, 32, 700, [32] * 32, 2048, torch.float16, "ragged"),
    ("rv8192_max_bf16", 1, 32, 8, 300, [64] * 8, 8192, torch.bfloat16, "ragged"),
    # more than 32 query heads: two P.V head groups (Llama-2-13B has 40 heads)
    ("mha_hq40", 2, 40, 40, 700, [96, 56, 48, 32, 16, 88, 56, 48] * 5, 1280, torch.float16, "ragged"),
    ("gqa_hq64_bf16", 1, 64, 8, 900, [32, 128, 32, 80, 32, 64, 80, 64], 512, torch.bfloat16, "ragged"),
    ("mha_hq64_s33", 2, 64, 64, 33, [16, 32] * 32, 200, torch.float16, "ragged"),
    # odd ranks (rows 2-byte aligned, repacked in 64-row blocks), GQA 4, and a
    # context that ends inside a block
    ("gqa4_odd_ranks", 2, 32, 8, 1000, [102, 37, 13, 70, 102, 5, 99, 128], 512, torch.float16, "ragged"),
]


@pytest.mark.parametrize("name,B,Hq,Hkv,S,ranks,Rv,dtype,layout", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle(name, B, Hq, Hkv, S, ranks, Rv, dtype, layout):
    ranks = ranks or cfg2_ranks()
    _flush(f"[decode] {name} B={B} Hq={Hq} Hkv={Hkv} S={S} Rv={Rv} {dtype}")
    case = make_case(B, Hq, Hkv, S, ranks, Rv, dtype=dtype, seed=1, layout=layout)
    ref, _, _ = oracle_decode(case)
    _check(case, ref)


def test_decode_llama3_rope_gqa_bf16():
    from starkv import RopeConfig
    rope = RopeConfig(theta=500000.0, rope_type="llama3", factor=8.0, low_freq_factor=1.0,
                      high_freq_factor=4.0, original_max_position_embeddings=8192)
    case = make_case(1, 32, 8, 9000, cfg4_ranks(), 512, dtype=torch.bfloat16, seed=2)
    _flush("[decode] llama3 gqa bf16 S=9000")
    ref, _, _ = oracle_decode(case, rope=rope)
    _check(case, ref, rope=rope)


def test_decode_attention_scaling_applied_once():
    """A RoPE attention scaling a != 1 multiplies cos and sin (HF
    LlamaRotaryEmbedding); the rotated query already carries one factor, the
    keys get theirs from the table, and the softmax scale is not multiplied
    again."""
    from starkv import RopeConfig
    rope = RopeConfig(attention_scaling=1.25)
    case = make_case(2, 32, 8, 700, cfg4_ranks(), 256, seed=5)
    _flush("[decode] attention_scaling 1.25")
    ref, _, _ = oracle_decode(case, rope=rope)
    _check(case, ref, rope=rope)


def test_decode_with_mask():
    case = make_case(2, 32, 32, 500, [32] * 32, 256, seed=3, layout="reference")
    mask = torch.zeros(2, 1, 1, 500, device="cuda", dtype=torch.float16)
    mask[0, ..., :100] = torch.finfo(torch.float16).min     # left padding of sequence 0
    mask[1, ..., 450:] = -5.0
    out = _run_decode(case, mask=mask)
    ref, _, _ = oracle_decode(case, mask=mask.float().view(2, 1, 500))
    mx, mr = errors(out, ref)
    assert mx <= MAX_ABS and mr <= MEAN_REL, (mx, mr)


def test_decode_with_mask_gqa():
    # 4 query heads per KV head: the grouped-query K-logit kernel, whose masked
    # form is a kernel of its own
    case = make_case(2, 32, 8, 700, cfg4_ranks(), 256, seed=11)
    mask = torch.zeros(2, 1, 1, 700, device="cuda", dtype=torch.float16)
    mask[0, ..., :130] = torch.finfo(torch.float16).min     # left padding of sequence 0
    mask[1, ..., 650:] = -5.0
    _flush("[decode] GQA with mask")
    out = _run_decode(case, mask=mask)
    ref, _, _ = oracle_decode(case, mask=mask.float().view(2, 1, 700))
    mx, mr = errors(out, ref)
    assert mx <= MAX_ABS and mr <= MEAN_REL, (mx, mr)


def test_decode_deterministic():
    case = make_case(4, 32, 32, 3000, cfg2_ranks(), 1640, seed=4)
    a = _run_decode(case).clone()
    b = _run_decode(case).clone()
    assert torch.equal(a, b)


def test_k_logits_matches_oracle():
    from starkv import RopeConfig, k_logits
    case = make_case(2, 32, 32, 1234, cfg2_ranks(), 64, seed=5)
    out = k_logits(case.q, case.kspec, case.S, RopeConfig(), scale=1.0)
    ref = oracle_logits(case)
    mx, mr = errors(out, ref)
    _flush(f"[k_logits] max_abs={mx:.3e} mean_rel={mr:.3e} ref_rms={ref.pow(2).mean().sqrt():.3f}")
    check_logits(out, ref, 1.0, "k_logits scale 1: ")


@pytest.mark.parametrize("Rv", [1640, 3000])
def test_pv_latent_matches_oracle(Rv):
    from starkv import pv_latent
    g = torch.Generator(device="cuda").manual_seed(6)
    B, H, S = 3, 32, 2000
    p = torch.softmax(torch.randn(B, H, S, device="cuda", generator=g), -1).half()
    xv = torch.randn(B, S, Rv, device="cuda", generator=g).half()
    out = pv_latent(p, xv)
    ref = p.double().cpu() @ xv.double().cpu()
    mx, mr = errors(out, ref)
    assert mr <= 1e-3 and mx <= 2e-2, (mx, mr)


@pytest.mark.parametrize("batch_sel", [[0], [15]])
def test_decode_cfg2_full_shape(batch_sel):
    """The benchmark workload itself (B16, S32768, ragged ranks sum 1640,
    Rv 1640, fp16): all 16 batches run on the GPU; the oracle (fp32 on the CPU)
    checks the selected batch."""
    case = make_case(16, 32, 32, 32768, cfg2_ranks(), 1640, seed=0)
    _flush(f"[decode] cfg2 full shape, checking batch {batch_sel}")
    out = _run_decode(case)
    ref, _, _ = oracle_decode(case, batches=batch_sel, dtype=torch.float32)
    mx, mr = errors(out[batch_sel], ref)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= MAX_ABS and mr <= MEAN_REL, (mx, mr)


@pytest.mark.parametrize("dtype,device_pos", [(torch.float16, False), (torch.bfloat16, True)])
def test_rope_apply_matches_oracle(dtype, device_pos):
    """The fused query rotation (model.py:423) against the oracle's apply_rope
    at positions pos0 + t, in place on a strided [B, H, T, 128] view; the
    position from the host or from a device int.  One rounding of the fp32
    result: within one unit in the last place of the act dtype."""
    from oracle import starkv_oracle as o
    from starkv import RopeConfig, rope_apply
    rope = RopeConfig(theta=500000.0, rope_type="llama3", factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                      original_max_position_embeddings=8192, attention_scaling=1.25)
    B, H, T, pos0 = 3, 8, 37, 1000
    g = torch.Generator(device="cuda").manual_seed(9)
    base = torch.randn(B, T, H, 128, generator=g, device="cuda").to(dtype)
    x = base.clone().transpose(1, 2)                                      # [B, H, T, 128], strided
    pos = torch.tensor([pos0], dtype=torch.int32, device="cuda") if device_pos else None
    rope_apply(x, rope, pos0=0 if device_pos else pos0, pos0_device=pos, max_positions=pos0 + T)
    torch.cuda.synchronize()
    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(pos0, pos0 + T), rope.attention_scaling)
    ref = o.apply_rope(base.transpose(1, 2).double().cpu(), cos.double(), sin.double())
    err = (x.double().cpu() - ref).abs()
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    assert float((err / ref.abs().clamp_min(1e-3)).max()) <= ulp or float(err.max()) <= ulp * 4, float(err.max())


@pytest.mark.gpu
@pytest.mark.parametrize("latent_scale,q_scale", [(30000.0, 1.0), (1.0, 1e5), (3000.0, 3e4)],
                         ids=["keys", "queries", "both"])
def test_k_logits_gqa_bf16_beyond_fp16_range(latent_scale, q_scale):
    """bf16 grouped-query K logits whose keys or queries exceed fp16's range
    (the reference holds them in bf16, abx_rope_batched.py:114-125): the
    grouped-query kernel's fp16 q.K step takes bf16 queries and keys scaled
    by 2^-8 (exact) and scales the logits back, so values up to 1.6e7 stay
    finite and the logits match the oracle relative to their own RMS
    (max-abs 2e-2, mean-rel 1e-3)."""
    from starkv import k_logits
    ranks = cfg4_ranks()
    case = make_case(1, 32, 8, 300, ranks, 512, dtype=torch.bfloat16, seed=41, latent_scale=latent_scale)
    case.q.mul_(q_scale)
    kmax = max(float((x.float() @ b.float()).abs().max()) for x, b in zip(case.xk_heads, case.bk_heads))
    qmax = float(case.q.float().abs().max())
    print(f"[k logits gqa bf16 large] max |K| before RoPE {kmax:.3e}, max |q| {qmax:.3e}", flush=True)
    assert max(kmax, qmax) > 65504.0
    out = k_logits(case.q, case.kspec, case.S)
    torch.cuda.synchronize()
    ref = oracle_logits(case)
    assert torch.isfinite(out).all()
    rms = float(ref.pow(2).mean().sqrt())
    mx, mr = errors(out / rms, ref / rms)
    print(f"   RMS {rms:.3e}: max_abs/RMS={mx:.3e} mean_rel={mr:.3e}", flush=True)
    assert mx <= 2e-2 and mr <= 1e-3


LAST_POS_CASES = [
    # name, B, Hq, Hkv, S, ranks, Rv, layout: each K-logit kernel family
    ("mha_ws_dense", 2, 32, 32, 700, None, 256, "ragged"),
    ("gqa4_dense", 2, 32, 8, 700, [32, 128, 32, 80, 32, 64, 80, 64], 256, "ragged"),
    ("unaligned_r_streaming", 2, 32, 32, 129, [20] * 32, 50, "reference"),
]


@pytest.mark.parametrize("name,B,Hq,Hkv,S,ranks,Rv,layout", LAST_POS_CASES, ids=[c[0] for c in LAST_POS_CASES])
def test_decode_last_pos_matches_additive_mask(name, B, Hq, Hkv, S, ranks, Rv, layout):
    """A device-held last position (positions after it at -1e30) gives the
    outputs of the additive -1e30 mask over the same positions, and both
    match the oracle."""
    from starkv import RopeConfig, decode_attention
    ranks = ranks or cfg2_ranks()
    _flush(f"[decode last_pos] {name}")
    case = make_case(B, Hq, Hkv, S, ranks, Rv, seed=21, layout=layout)
    last = S - 1 - S // 5
    mask = torch.zeros(B, 1, S, device="cuda", dtype=torch.float32)
    mask[..., last + 1:] = -1e30
    lp = torch.tensor([last], dtype=torch.int32, device="cuda")
    rope = RopeConfig()
    a = decode_attention(case.q, case.kspec, case.xv, case.uv, rope=rope, last_pos=lp)
    m = decode_attention(case.q, case.kspec, case.xv, case.uv, rope=rope, mask=mask)
    ref, _, _ = oracle_decode(case, mask=mask.double().cpu())
    mx, mr = errors(a, m.float())
    _flush(f"   last_pos vs mask: max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= 1e-3 and mr <= 1e-5, (mx, mr)
    mx, mr = errors(a, ref)
    _flush(f"   last_pos vs oracle: max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= MAX_ABS and mr <= MEAN_REL, (mx, mr)


def test_decode_last_pos_int8_k_cache():
    """The same over the int8-K / int4-g64-V cache the e2e harness decodes
    from: the warp-specialised int8 K-logit kernel takes its pipelined loop
    under last_pos and its mask loop under the additive mask."""
    from starkv import RopeConfig, decode_attention
    from starkv.cache import LatentCache
    _flush("[decode last_pos] int8 K cache")
    ranks, B, S, Rv = cfg2_ranks(), 2, 1500, 1640
    H, rmax = len(ranks), max(ranks)
    g = torch.Generator(device="cuda").manual_seed(22)
    k_new = torch.randn(B, H, S, rmax, generator=g, device="cuda").half()
    v_new = torch.randn(B, S, Rv, generator=g, device="cuda").half()
    bk = (torch.randn(H, rmax, HEAD_DIM_T, generator=g, device="cuda") / math.sqrt(rmax)).half()
    uv = (torch.randn(H * HEAD_DIM_T, Rv, generator=g, device="cuda") / math.sqrt(Rv)).half()
    q = torch.randn(B, H, HEAD_DIM_T, generator=g, device="cuda").half()
    cache = LatentCache(B, ranks, Rv, S + 7, torch.float16, "cuda", fmt="int8_g64")
    kspec, vspec, _ = cache.append(k_new, v_new, bk)
    cap = S + 7
    last = S - 1
    mask = torch.zeros(B, 1, cap, device="cuda", dtype=torch.float32)
    mask[..., last + 1:] = -1e30
    lp = torch.tensor([last], dtype=torch.int32, device="cuda")
    rope = RopeConfig()
    a = decode_attention(q, kspec, vspec, uv, rope=rope, seq_len=cap, last_pos=lp)
    m = decode_attention(q, kspec, vspec, uv, rope=rope, seq_len=cap, mask=mask)
    e = decode_attention(q, kspec, vspec, uv, rope=rope, seq_len=S)
    for nm, other in (("mask", m), ("length", e)):
        mx, mr = errors(a, other.float())
        _flush(f"   last_pos vs {nm}: max_abs={mx:.3e} mean_rel={mr:.3e}")
        assert mx <= 2e-3 and mr <= 1e-4, (nm, mx, mr)
