"""GPU checks of the e2e decoder layer's elementwise kernels (starkv_rms_norm,
starkv_silu_mul) against the HF / torch operations they replace, and of the
fused decoder layer against HF's own layer forward.

torch rounds to the activation dtype after each of HF's operations; the
kernels round at the same points, so the outputs agree to within one unit in
the last place of an intermediate (the fp32 sum of squares is taken in
another order, and rsqrt / exp are the device's), i.e. at most 2 in the
output after the last multiply, and the residual sum x + residual is exact
(two fp16 / bf16 values add exactly in fp32 before the one rounding)."""
import sys

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ulp(dtype):
    return 10 if dtype == torch.float16 else 7        # significand bits after the leading one


def _ulps_dt(a, b, dtype):
    """Largest |a - b| in units in the last place of the larger of |a|, |b|
    (dtype's precision; values below 2^-14 count at 2^-14); prints the share
    of elements that differ."""
    a64, b64 = a.detach().cpu().double(), b.detach().cpu().double()
    _, e = torch.frexp(torch.maximum(a64.abs(), b64.abs()).clamp_min(2.0 ** -14))   # x = m 2^e, m in [0.5, 1)
    d = (a64 - b64).abs()
    _flush(f"   {float((d > 0).double().mean()) * 100:.3f} % of elements differ")
    return float((d / torch.ldexp(torch.ones_like(d), e - 1 - _ulp(dtype))).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,hidden", [(8, 4096), (3, 1024), (513, 4096), (2, 16384), (5, 40)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rms_norm_matches_hf(dtype, rows, hidden, with_residual):
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    from starkv.ops import rms_norm
    _flush(f"[rms_norm] rows={rows} hidden={hidden} {dtype} residual={with_residual}")
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + hidden)
    x = (torch.randn(rows, hidden, generator=g, device="cuda") * 3).to(dtype)
    res = (torch.randn(rows, hidden, generator=g, device="cuda") * 3).to(dtype)
    mod = LlamaRMSNorm(hidden, eps=1e-5).to(device="cuda", dtype=dtype)
    mod.weight.data.normal_(1.0, 0.2, generator=g)
    xin = x + res if with_residual else x
    ref = mod(xin)
    if with_residual:
        res_out = torch.empty_like(x)
        out = rms_norm(x, mod.weight, 1e-5, residual=res, residual_out=res_out)
        assert torch.equal(res_out, xin)
    else:
        out = rms_norm(x, mod.weight, 1e-5)
    torch.cuda.synchronize()
    u = _ulps_dt(out, ref, dtype)
    _flush(f"   max {u:.2f} ulp")
    assert u <= 2.0


def test_rms_norm_in_place_and_strided():
    """out aliasing x, and rows addressed with a stride (a column slice of a wider tensor)."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    from starkv.ops import rms_norm
    g = torch.Generator(device="cuda").manual_seed(9)
    wide = torch.randn(2, 7, 4096 + 512, generator=g, device="cuda").half()
    x = wide[..., :4096]
    mod = LlamaRMSNorm(4096, eps=1e-6).to(device="cuda", dtype=torch.float16)
    ref = mod(x.contiguous())
    out = rms_norm(x, mod.weight, 1e-6)
    assert _ulps_dt(out, ref, torch.float16) <= 2.0
    y = x.contiguous()
    rms_norm(y, mod.weight, 1e-6, out=y)
    torch.cuda.synchronize()
    assert torch.equal(y, out)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,width", [(8, 11008), (1, 8), (1000, 2048)])
def test_silu_mul_matches_torch(dtype, rows, width):
    from starkv.ops import silu_mul
    _flush(f"[silu_mul] rows={rows} width={width} {dtype}")
    g = torch.Generator(device="cuda").manual_seed(rows + width)
    gu = (torch.randn(rows, 2 * width, generator=g, device="cuda") * 4).to(dtype)
    ref = F.silu(gu[:, :width]) * gu[:, width:]
    out = silu_mul(gu)
    out2 = silu_mul(gu[:, :width], gu[:, width:])
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    u = _ulps_dt(out, ref, dtype)
    _flush(f"   max {u:.2f} ulp")
    assert u <= 2.0


GEMM_CASES = [
    # m, n, k, epilogue, dtype
    (8, 7376, 4096, 0, torch.float16), (8, 4096, 4096, 1, torch.float16), (8, 22016, 4096, 2, torch.float16),
    (8, 4096, 11008, 1, torch.float16), (1, 256, 64, 0, torch.float16), (16, 512, 1088, 0, torch.bfloat16),
    (3, 1024, 2048, 2, torch.bfloat16), (13, 2048, 704, 1, torch.bfloat16), (8, 32000, 4096, 0, torch.float16),
    (9, 96, 192, 2, torch.float16),
]


@pytest.mark.parametrize("mode", ["rowmajor", "packed", "packed_rms"])
@pytest.mark.parametrize("case", GEMM_CASES, ids=[f"m{c[0]}n{c[1]}k{c[2]}e{c[3]}{str(c[4])[-4:]}" for c in GEMM_CASES])
def test_skinny_gemm_matches_fp32(case, mode):
    """starkv_skinny_gemm against the fp32 product rounded as torch rounds it:
    epilogue 0 act(x W^T); 1 act(x W^T + out); 2 act(act(silu(act(g))) act(u)).
    The fp32 sums run in another order than the reference's, so the gate is
    one rounding of the output plus the fp32 accumulation error
    (k 2^-24 sum |x||w|).  "packed": the weight in pack_weight's layout (the
    same results); "packed_rms": x is an RMSNorm's raw input, the norm
    weight folded into the packed weight, and the reference product is
    (x rsqrt(mean(x^2) + eps)) act(W nw)^T."""
    from starkv.ops import pack_weight, skinny_linear
    m, n, k, epi, dtype = case
    _flush(f"[skinny gemm] m={m} n={n} k={k} epilogue={epi} {dtype} {mode}")
    g = torch.Generator(device="cuda").manual_seed(m * 31 + n + k)
    x = torch.randn(m, k, generator=g, device="cuda").to(dtype)
    w = (torch.randn(n, k, generator=g, device="cuda") / k ** 0.5).to(dtype)
    eps = 1e-5
    if mode == "packed_rms":
        nw = (1.0 + 0.2 * torch.randn(k, generator=g, device="cuda")).to(dtype)
        wk = pack_weight(w, nw)
        wf = (w.float() * nw.float()).to(dtype).double()
        xd = x.double() * torch.rsqrt(x.double().pow(2).mean(-1, keepdim=True) + eps)
    else:
        wk = pack_weight(w) if mode == "packed" else w
        wf, xd = w.double(), x.double()
    acc = xd @ wf.t()
    bound = k * 2.0 ** -24 * (xd.abs() @ wf.abs().t())
    lin = (lambda xx, **kw: skinny_linear(xx, wk, rms_eps=eps if mode == "packed_rms" else None, **kw))
    if epi == 2:
        h = n // 2
        gt, up = acc[:, :h].to(dtype), acc[:, h:].to(dtype)
        ref = (F.silu(gt.float()).to(dtype).double() * up.double())
        out = lin(x, epilogue=2)
        bound = 4 * bound[:, :h] + 2.0 ** -8 * ref.abs()          # two roundings of the inputs feed the product
    elif epi == 1:
        res = torch.randn(m, n, generator=g, device="cuda").to(dtype)
        ref = acc + res.double()
        out = res.clone()
        lin(x, out=out, epilogue=1)
    else:
        ref = acc
        out = lin(x)
    torch.cuda.synchronize()
    ulp = 2.0 ** -(10 if dtype == torch.float16 else 7)
    err = (out.double() - ref).abs()
    lim = bound + ulp * ref.abs() + 2.0 ** -24
    worst = float((err / lim).max())
    _flush(f"   worst error / bound = {worst:.3f}")
    assert worst <= 1.0


@pytest.mark.parametrize("T", [1, 37])
def test_fused_decoder_layer_matches_hf_forward(T):
    """One decoder layer of the e2e model through the fused forward against
    HF's own LlamaDecoderLayer.forward on the same weights and caches: the
    layer outputs within max-abs 2e-2 and mean-rel 1e-3 (the residual adds
    round once inside the GEMMs instead of twice; at T = 1 the RMSNorms are
    folded into the projections, so the normalised input is not rounded).
    Dense latent caches: quantising the new latents would turn last-place
    differences of the projections into whole quantisation steps."""
    import starkv.e2e as e2e
    from _util import errors
    _flush(f"[fused layer] T={T}")
    kw = dict(n_layers=1, hidden=1024, heads=8, kv_heads=2, intermediate=2048, vocab=1000, ranks=[48, 96],
              v_rank=256, batch=2, capacity=64, fmt="dense", seed=7)
    fused, plain = e2e.build_model(**kw), e2e.build_model(**kw, fused=False)
    for a, b in zip(fused.state_dict().values(), plain.state_dict().values()):
        assert torch.equal(a, b)
    g = torch.Generator(device="cuda").manual_seed(8)
    h = (torch.randn(2, T, 1024, generator=g, device="cuda")).half()
    outs = []
    for m in (fused, plain):
        layer = m.model.layers[0]
        pos = torch.arange(T, device="cuda")[None].expand(2, T)
        pe = m.model.rotary_emb(h, pos)
        with torch.no_grad():
            # the fused forward updates its input (the residual stream) in place
            outs.append(layer(h.clone(), attention_mask=None, position_ids=pos, position_embeddings=pe))
    torch.cuda.synchronize()
    mx, mr = errors(outs[0], outs[1])
    _flush(f"   max_abs={mx:.3e} mean_rel={mr:.3e}")
    assert mx <= 2e-2 and mr <= 1e-3
