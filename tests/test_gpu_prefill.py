"""GPU parity of the causal prefill over the latent caches
(starkv_prefill_attention; the reference's prefill branch model.py:429-449
under a causal mask) against the CPU oracle's prefill_attention.

Inputs are rounded to the act dtype first and the oracle runs in float64 on
those values (quantised latents: on the oracle-dequantised fp16 values,
rounded to bf16 for bf16 cases, as the kernel dequantises).  The reference
materialises K and V in the act dtype (model.py:431-442); the kernel holds
them in fp16 for both act dtypes (finer than bf16): the oracle rounds its
fp64 K (after RoPE) and V once to fp16, then attends in fp64.  Gates: max-abs
2e-2 and mean-rel 1e-3 (bf16 outputs against the bf16-rounded oracle).
"""
import math
import sys

import numpy as np
import pytest
import torch

from _util import check_output, errors

HEAD = 128


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dense_k(B, S, ranks, dtype, g):
    """Ragged dense K latent: one buffer [B, S*sum(r)], head h at S*cumsum(r)[h]."""
    from starkv import KLatentSpec
    per_b = S * sum(ranks)
    buf = torch.randn(B, per_b, generator=g, device="cuda").to(dtype)
    offs = list(np.cumsum([0] + ranks[:-1]) * S)
    heads = [buf[:, o:o + S * r].view(B, S, r) for o, r in zip(offs, ranks)]
    return buf, offs, heads


def _bk(ranks, dtype, g):
    bk_all = torch.empty(sum(ranks), HEAD, device="cuda")
    bko, heads, row = [], [], 0
    for r in ranks:
        bk_all[row:row + r] = torch.randn(r, HEAD, generator=g, device="cuda") / math.sqrt(r)
        bko.append(row * HEAD)
        row += r
    bk_all = bk_all.to(dtype)
    row = 0
    for r in ranks:
        heads.append(bk_all[row:row + r])
        row += r
    return bk_all, bko, heads


def _run(B, Hq, ranks, Rv, T, pos0, dtype, kfmt="dense", vfmt="dense", seed=0, rope=None):
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, RopeConfig, prefill_attention
    from starkv._lib import FMT_INT8_SYM
    _flush(f"[prefill] B={B} Hq={Hq} Hkv={len(ranks)} T={T} pos0={pos0} Rv={Rv} {dtype} K={kfmt} V={vfmt}")
    g = torch.Generator(device="cuda").manual_seed(seed)
    Hkv = len(ranks)
    S = pos0 + T
    bk_all, bko, bk_heads = _bk(ranks, dtype, g)
    if kfmt == "dense":
        buf, offs, xk_dev = _dense_k(B, S, ranks, dtype, g)
        kspec = KLatentSpec(buf, ranks, offs, ranks, buf.stride(0), bk_all, bko, HEAD)
        xk = [x.double().cpu() for x in xk_dev]
    elif kfmt.startswith("ref"):
        # the reference module's split K cache (uniform rank): "ref8_U" / "ref4_U" = an int8 / int4
        # upper block of U ranks over an int4 lower one, "ref4w" = all ranks int4
        from test_gpu_quant_k import reference_split_k
        r = ranks[0]
        assert ranks == [r] * Hkv
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        bk = bk_all.view(Hkv, r, HEAD)
        if kfmt == "ref4w":
            q1, s1, _, _, deq = reference_split_k(B, Hkv, S, r, 0, "int4", seed=seed + 1)
            kspec = KLatentSpec.from_reference_quant(dev(q1), dev(s1), bk, r)
        else:
            up = int(kfmt.split("_")[1])
            q1, s1, q2, s2, deq = reference_split_k(B, Hkv, S, up, r - up, "int8" if kfmt[3] == "8" else "int4",
                                                    seed=seed + 1)
            kspec = KLatentSpec.from_reference_quant(dev(q1), dev(s1), bk, r, x2=dev(q2), s2=dev(s2), split=up)
        xk = [torch.from_numpy(deq[:, h]).to(dtype).double() for h in range(Hkv)]
    else:
        from test_gpu_quant_k import ragged_int8_k
        kb, scales, offs, deq = ragged_int8_k(B, S, ranks, seed=seed + 1)
        sc = torch.from_numpy(scales).cuda()
        kspec = KLatentSpec(torch.from_numpy(kb).cuda(), ranks, offs, ranks, kb.shape[1], bk_all, bko, HEAD,
                            fmt=FMT_INT8_SYM, scale=sc, scale_stride_b=sc.stride(0), scale_stride_h=sc.stride(1))
        xk = [d.to(dtype).double() for d in deq]
    if vfmt == "dense":
        xv_dev = torch.randn(B, S, Rv, generator=g, device="cuda").to(dtype)
        v = xv_dev
        xv = xv_dev.double().cpu()
    else:
        # "g64", or a per-token block kind of make_quant_v ("ref_int4" / "ref_int8" with the upper
        # block's width after a colon, "int8", "int4_whole")
        from test_gpu_quant import make_quant_v
        kind, _, split = vfmt.partition(":")
        v, dq, _ = make_quant_v(kind, B, S, Rv, split=int(split or 256), seed=seed + 2)
        xv = torch.from_numpy(dq.astype(np.float64)).to(dtype).double()
    uv = (torch.randn(Hkv * HEAD, Rv, generator=g, device="cuda") / math.sqrt(Rv)).to(dtype)
    q = torch.randn(B, Hq, T, HEAD, generator=g, device="cuda").to(dtype)
    rope = rope or RopeConfig()
    out = prefill_attention(q, kspec, v, uv, rope=rope, pos0=pos0)
    torch.cuda.synchronize()
    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), rope.attention_scaling)
    ref = o.prefill_attention(q.double().cpu(), [b.double().cpu() for b in bk_heads], xk, xv, uv.double().cpu(),
                              cos.double(), sin.double(), pos0=pos0, kv_dtype=torch.float16)
    check_output(out, ref)
    return out


CASES = [
    # name, B, Hq, ranks, Rv, T, pos0, dtype, K format, V format
    ("mha_ragged_f16", 2, 4, [8, 24, 64, 128], 96, 200, 0, torch.float16, "dense", "dense"),
    ("gqa4_bf16", 2, 8, [32, 80], 160, 300, 0, torch.bfloat16, "dense", "dense"),
    ("chunk_pos0", 1, 8, [16, 40], 64, 77, 150, torch.float16, "dense", "dense"),
    ("one_token", 2, 4, [24, 8, 128, 56], 40, 1, 500, torch.float16, "dense", "dense"),
    ("t1024_f16", 1, 2, [48, 128], 256, 1024, 0, torch.float16, "dense", "dense"),
    ("int8k_g64v_f16", 2, 4, [64, 32, 96, 128], 200, 129, 0, torch.float16, "int8", "g64"),
    ("int8k_g64v_bf16_chunk", 1, 8, [32, 128], 1640, 96, 64, torch.bfloat16, "int8", "g64"),
    # an odd KV-head count leaves the last V head pair half empty; MQA has one KV head
    ("odd_hkv3_gqa2", 2, 6, [24, 64, 40], 72, 130, 5, torch.float16, "dense", "dense"),
    ("mqa_int8_g64", 1, 8, [96], 136, 300, 0, torch.float16, "int8", "g64"),
    # the reference module's quantised caches: split K (int8 / int4 upper block over int4) and
    # per-token block V (int8 / int4 upper block over int4, whole int8, whole int4)
    ("ref8k_ref8v_f16", 2, 8, [80, 80], 512, 150, 0, torch.float16, "ref8_16", "ref_int8:256"),
    ("ref8k_ref4v_bf16_chunk", 1, 8, [128] * 4, 384, 100, 37, torch.bfloat16, "ref8_16", "ref_int4:256"),
    ("ref4k_int8v_mha", 2, 4, [64] * 4, 264, 129, 0, torch.float16, "ref4_32", "int8"),
    ("ref4w_k_int4w_v", 1, 4, [48] * 2, 512, 257, 3, torch.bfloat16, "ref4w", "int4_whole"),
    ("ref8k_ref8v_cfg_ranks", 1, 32, [128] * 8, 1640, 64, 200, torch.float16, "ref8_16", "ref_int8:256"),
    # ranks that are not multiples of 8 and rows of any alignment (repacked into aligned workspace
    # rows first): dense K heads back to back, V rank 60 (U_v rows of 60 columns too), int8 K of odd
    # ranks with group-64 V of rank 1229, the reference module's K at rank 100 over the bx default
    # V rank 1228 (486-byte lower rows), whole-rank int4 K and V of odd ranks, int8 V of rank 77
    ("dense_any_rank", 2, 4, [20, 37, 5, 128], 60, 150, 10, torch.float16, "dense", "dense"),
    ("int8k_g64v_any_rank_bf16", 1, 8, [37, 100], 1229, 120, 0, torch.bfloat16, "int8", "g64"),
    ("ref8k_r100_ref4v_r1228", 1, 8, [100, 100], 1228, 100, 20, torch.float16, "ref8_16", "ref_int4:256"),
    ("ref4w_k_int4w_v_odd", 1, 4, [75, 75], 203, 97, 0, torch.float16, "ref4w", "int4_whole"),
    ("int8k_int8v_odd", 2, 4, [33, 17], 77, 64, 3, torch.bfloat16, "int8", "int8"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_prefill_matches_oracle(case):
    _run(*case[1:])


@pytest.mark.gpu
def test_prefill_llama3_rope_attention_scaling():
    """llama3 inverse frequencies and an attention scaling != 1 (applied once,
    through the keys' RoPE table), chunked, GQA."""
    from starkv import RopeConfig
    rope = RopeConfig(theta=500000.0, rope_type="llama3", factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                      original_max_position_embeddings=8192, attention_scaling=1.25)
    _run(1, 8, [32, 128], 96, 150, 260, torch.float16, rope=rope)


@pytest.mark.gpu
def test_prefill_last_row_matches_decode():
    """The last prefill query is the decode step over the same caches."""
    from starkv import KLatentSpec, RopeConfig, decode_attention, prefill_attention
    _flush("[prefill] last row vs decode")
    g = torch.Generator(device="cuda").manual_seed(7)
    B, Hq, ranks, Rv, T = 2, 8, [40, 104], 120, 333
    bk_all, bko, _ = _bk(ranks, torch.float16, g)
    buf, offs, _ = _dense_k(B, T, ranks, torch.float16, g)
    kspec = KLatentSpec(buf, ranks, offs, ranks, buf.stride(0), bk_all, bko, HEAD)
    xv = torch.randn(B, T, Rv, generator=g, device="cuda").half()
    uv = (torch.randn(len(ranks) * HEAD, Rv, generator=g, device="cuda") / math.sqrt(Rv)).half()
    q = torch.randn(B, Hq, T, HEAD, generator=g, device="cuda").half()
    pre = prefill_attention(q, kspec, xv, uv, rope=RopeConfig())
    dec = decode_attention(q[:, :, -1].contiguous(), kspec, xv, uv, rope=RopeConfig(), out_dtype=torch.float32)
    mx, mr = errors(pre[:, :, -1], dec)
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= 2e-2 and mr <= 2e-3, (mx, mr)


@pytest.mark.gpu
@pytest.mark.parametrize("B,T", [(2, 8192), (1, 16384), (1, 32768)])
def test_prefill_e2e_shape_sampled_rows(B, T):
    """The e2e workload's prefill layer at full prompt length (8192 tokens)
    and at the longer contexts the reference's e2e sweep reaches (latency.py:
    353-357): MHA 32 x 128, the cfg2 ragged K ranks (sum 1640) as int8 per
    (b, h, s), V rank 1640 as int4 group-64, fp16.  The whole prompt runs on
    the GPU; sampled query rows are checked against the oracle's prefill of
    that row alone (pos0 = t: the decode step over the first t + 1 positions,
    pinned on the CPU by the oracle's chunk / last-row identities) as the
    reference computes it for an fp16 model: cos / sin cast to fp16 (HF's
    rotary embedding returns them in the activations' dtype) and K, V
    materialised in fp16 (model.py:431-442), then fp64 attention.  The error
    against fp32 cos / sin with fp64 K, V is printed beside it: those two
    fp16 roundings, which the reference shares, put ~7e-4 mean-rel between
    the two oracles at 16K positions (CPU emulation of the kernel's steps:
    7e-5 from the first, 7.6e-4 from the second)."""
    from oracle import starkv_oracle as o
    from starkv import KLatentSpec, RopeConfig, prefill_attention
    from starkv._lib import FMT_INT8_SYM
    from test_gpu_quant import make_quant_v
    from test_gpu_quant_k import ragged_int8_k
    from _util import cfg2_ranks
    Rv = 1640
    ranks = cfg2_ranks()
    Hkv = Hq = len(ranks)
    _flush(f"[prefill e2e shape] B={B} T={T} Hq={Hq} ranks sum {sum(ranks)} int8 K, Rv={Rv} g64 V")
    g = torch.Generator(device="cuda").manual_seed(21)
    bk_all, bko, bk_heads = _bk(ranks, torch.float16, g)
    kb, scales, offs, deq_k = ragged_int8_k(B, T, ranks, seed=22)
    sc = torch.from_numpy(scales).cuda()
    kspec = KLatentSpec(torch.from_numpy(kb).cuda(), ranks, offs, ranks, kb.shape[1], bk_all, bko, HEAD,
                        fmt=FMT_INT8_SYM, scale=sc, scale_stride_b=sc.stride(0), scale_stride_h=sc.stride(1))
    vspec, deq_v, _ = make_quant_v("g64", B, T, Rv, seed=23)
    uv = (torch.randn(Hkv * HEAD, Rv, generator=g, device="cuda") / math.sqrt(Rv)).half()
    q = torch.randn(B, Hq, T, HEAD, generator=g, device="cuda").half()
    rope = RopeConfig()
    out = prefill_attention(q, kspec, vspec, uv, rope=rope)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(T), rope.attention_scaling)
    xv = torch.from_numpy(deq_v.astype(np.float64))
    bk = [b.double().cpu() for b in bk_heads]
    uvd = uv.double().cpu()
    for b, t in [(0, 0), (B - 1, 1), (0, 777), (B - 1, 4095), (0, T // 2 + 17), (B - 1, T - 1)]:
        S = t + 1
        qt = q[b:b + 1, :, t:t + 1].double().cpu()
        xks = [x[b:b + 1, :S] for x in deq_k]
        ref64 = o.prefill_attention(qt, bk, xks, xv[b:b + 1, :S], uvd, cos.double()[:S], sin.double()[:S], pos0=t)
        mx64, mr64 = errors(out[b:b + 1, :, t], ref64[:, :, 0])
        _flush(f"   b={b} t={t}: against fp64 K / V: max_abs={mx64:.3e} mean_rel={mr64:.3e}")
        ref = o.prefill_attention(qt, bk, xks, xv[b:b + 1, :S], uvd, cos.half().double()[:S],
                                  sin.half().double()[:S], pos0=t, kv_dtype=torch.float16)
        check_output(out[b:b + 1, :, t], ref[:, :, 0], f"b={b} t={t} (fp16 cos / sin, K, V: the reference's): ")
