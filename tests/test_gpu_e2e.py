"""GPU test of the end-to-end decode harness (starkv.e2e): a small random-init
Llama-shaped model whose attentions prefill and decode on the HIP kernels over
quantised latent caches, against the same model running every forward through
the torch path (dequantised caches, K / V materialised, SDPA), fed the same
tokens."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("kv_heads,ranks,fmt", [(8, [32, 48, 16, 64, 32, 56, 16, 96], "int8_g64"),
                                                (2, [48, 96], "int8_g64"),
                                                (8, [32, 48, 16, 64, 32, 56, 16, 96], "dense")])
def test_e2e_decode_matches_torch_path(kv_heads, ranks, fmt):
    from starkv.e2e import build_model, generate
    _flush(f"[e2e] layers=2 hidden=1024 kv_heads={kv_heads} fmt={fmt}")
    B, P, steps = 2, 40, 4
    kw = dict(n_layers=2, hidden=1024, heads=8, kv_heads=kv_heads, intermediate=2048, vocab=1000, ranks=ranks,
              v_rank=256, batch=B, capacity=P + steps + 1, fmt=fmt, seed=3)
    g = torch.Generator(device="cuda").manual_seed(5)
    prompt = torch.randint(0, 1000, (B, P), generator=g, device="cuda")
    model = build_model(**kw)
    toks, logits = generate(model, prompt, steps)
    torch.cuda.synchronize()
    ref_model = build_model(**kw)
    _, ref_logits = generate(ref_model, prompt, steps, reference=True, forced=toks[:, :steps])
    torch.cuda.synchronize()
    for t, (a, r) in enumerate(zip(logits, ref_logits)):
        d = (a.double() - r.double()).abs()
        mr = float(d.mean() / r.double().abs().mean())
        _flush(f"   forward {t}: max_abs={float(d.max()):.3e} mean_rel={mr:.3e}")
        assert torch.isfinite(a).all()
        assert mr <= 1e-2, (t, mr)


@pytest.mark.parametrize("fmt", ["int8_g64", "dense"])
def test_e2e_graph_replay_matches_eager(fmt):
    """Decode steps replayed from one captured graph (device-side cache
    position, masked full-capacity attention) against the same model decoding
    eagerly on the kernels, fed the same tokens: every replay's logits close to
    the eager step's, the greedy tokens equal."""
    from starkv.e2e import build_model, generate, generate_graphed
    _flush(f"[e2e graph] fmt={fmt}")
    B, P, steps = 2, 40, 6
    kw = dict(n_layers=2, hidden=1024, heads=8, kv_heads=2, intermediate=2048, vocab=1000, ranks=[48, 96],
              v_rank=256, batch=B, capacity=P + steps + 3, fmt=fmt, seed=4)
    prompt = torch.randint(0, 1000, (B, P), generator=torch.Generator(device="cuda").manual_seed(6), device="cuda")
    model = build_model(**kw)
    toks, logits = generate_graphed(model, prompt, steps)
    torch.cuda.synchronize()
    ref_model = build_model(**kw)
    ref_toks, ref_logits = generate(ref_model, prompt, steps, forced=toks[:, :steps])
    torch.cuda.synchronize()
    assert len(logits) == steps + 1
    for t, (a, r) in enumerate(zip(logits, ref_logits)):
        d = (a.double() - r.double()).abs()
        mr = float(d.mean() / r.double().abs().mean())
        _flush(f"   forward {t}: max_abs={float(d.max()):.3e} mean_rel={mr:.3e}")
        assert torch.isfinite(a).all()
        assert mr <= 2e-3, (t, mr)
    assert torch.equal(toks, ref_toks)
    assert all(a.cache.length == P + steps for a in model.model.layers and [l.self_attn for l in model.model.layers])


def _random_export(g, hidden, kv_heads, keep, v_keep):
    """A layer's trained decomposition with orthonormal factors and thresholds
    that keep `keep[h]` K ranks per head and `v_keep` V ranks, exported with
    the reference's state-dict keys (model.py:76-205, 286-362)."""
    from starkv.export import export_state_dict
    D = 128

    def orth(n, k):
        q, _ = torch.linalg.qr(torch.randn(n, k, generator=g, dtype=torch.float64))
        return q[:, :k]

    sd = {}
    sig = torch.linspace(2.0, 0.02, D)
    U = torch.zeros(kv_heads * D, kv_heads * D, dtype=torch.float64)
    V = torch.zeros(kv_heads * D, hidden, dtype=torch.float64)
    for h in range(kv_heads):
        U[h * D:(h + 1) * D, h * D:(h + 1) * D] = orth(D, D)
        V[h * D:(h + 1) * D] = orth(hidden, D).t()
        sd[f"k_proj.Sigma_blocks.{h}.diag"] = sig
        sd[f"k_proj.Sigma_blocks.{h}.soft_thres_layer.alpha"] = torch.tensor([float(sig[keep[h]])])
    sd["k_proj.U.weight"], sd["k_proj.V.weight"] = U.float(), V.float()
    rv = 512
    sv = torch.linspace(1.5, 0.01, rv)
    sd["v_proj.U.weight"] = orth(kv_heads * D, rv).float()
    sd["v_proj.V.weight"] = orth(hidden, rv).t().float()
    sd["v_proj.Sigma.diag"] = sv
    sd["v_proj.Sigma.soft_thres_layer.alpha"] = torch.tensor([float(sv[v_keep])])
    p = export_state_dict(sd, dtype=torch.float16)
    for name in ("k_vs", "bk", "v_vs", "v_u"):
        setattr(p, name, getattr(p, name).cuda())
    return p


@pytest.mark.parametrize("fmt", ["int8_g64", "dense"])
def test_e2e_decode_over_exported_ragged_projections(fmt):
    """Layers built from exported trained decompositions (ragged kept ranks,
    padded to multiples of 8) decode on the HIP kernels as the torch path does."""
    from starkv.e2e import build_model, generate
    _flush(f"[e2e export] fmt={fmt}")
    g = torch.Generator().manual_seed(11)
    keeps = [[37, 70, 12, 101, 33, 64, 5, 120], [90, 16, 48, 127, 3, 60, 77, 25]]
    proj = [_random_export(g, 1024, 8, k, 300 + 11 * i) for i, k in enumerate(keeps)]
    for p in proj:
        assert all(r % 8 == 0 for r in p.ranks) and p.v_vs.shape[0] % 8 == 0
    B, P, steps = 2, 40, 4
    kw = dict(n_layers=2, hidden=1024, heads=8, kv_heads=8, intermediate=2048, vocab=1000, ranks=None,
              v_rank=None, batch=B, capacity=P + steps + 1, fmt=fmt, seed=3, projections=proj)
    prompt = torch.randint(0, 1000, (B, P), generator=torch.Generator(device="cuda").manual_seed(5), device="cuda")
    model = build_model(**kw)
    toks, logits = generate(model, prompt, steps)
    torch.cuda.synchronize()
    ref_model = build_model(**kw)
    _, ref_logits = generate(ref_model, prompt, steps, reference=True, forced=toks[:, :steps])
    torch.cuda.synchronize()
    for t, (a, r) in enumerate(zip(logits, ref_logits)):
        d = (a.double() - r.double()).abs()
        mr = float(d.mean() / r.double().abs().mean())
        _flush(f"   forward {t}: max_abs={float(d.max()):.3e} mean_rel={mr:.3e}")
        assert torch.isfinite(a).all()
        assert mr <= 1e-2, (t, mr)
