"""GPU test of the end-to-end decode harness (starkv.e2e): a small random-init
Llama-shaped model whose attentions decode on the HIP kernels over
quantised latent caches, against the same model decoding every step through
the torch path (dequantised caches, fp32 SDPA), fed the same tokens.  Both
runs prefill the same way, so their caches start identical."""
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
        if t == 0:
            assert torch.equal(a, r)               # same prefill path, same caches
        assert mr <= 1e-2, (t, mr)
