"""GPU tests of the end-to-end decode harness (starkv.e2e): random-init
Llama-shaped models whose attentions prefill and decode on the HIP kernels
over latent caches.

Parity gate: every attention call the model makes (the causal prefill and
each decode step, every layer) is recorded and its output checked against
the fp64 oracle run on the same inputs -- the rotated queries and the caches
as the writer stored them, dequantised bit-exactly -- at max-abs 2e-2 and
mean-rel 1e-3.  (The cache writer itself is checked bit-exactly against the
oracle's quantisers in test_gpu_cache.py.)  Graph-replayed decoding is checked
against eager decoding on the same kernels."""
import sys

import pytest
import torch

from _util import KernelRecorder, cfg2_ranks, errors

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _compare_logits(logits, ref_logits, tol):
    for t, (a, r) in enumerate(zip(logits, ref_logits)):
        d = (a.double() - r.double()).abs()
        mr = float(d.mean() / r.double().abs().mean())
        _flush(f"   model logits, forward {t}: max_abs={float(d.max()):.3e} mean_rel={mr:.3e}")
        assert torch.isfinite(a).all()
        assert mr <= tol, (t, mr)


SHAPES = [
    # name, layers, hidden, heads, kv_heads, MLP, vocab, ranks, Rv, fmt, batch, prompt, steps
    ("gqa8_int8_g64", 2, 1024, 8, 8, 2048, 1000, [32, 48, 16, 64, 32, 56, 16, 96], 256, "int8_g64", 2, 40, 4),
    ("gqa2_int8_g64", 2, 1024, 8, 2, 2048, 1000, [48, 96], 256, "int8_g64", 2, 40, 4),
    ("gqa8_dense", 2, 1024, 8, 8, 2048, 1000, [32, 48, 16, 64, 32, 56, 16, 96], 256, "dense", 2, 40, 4),
    # the e2e workload's layer shape: Llama-2-7B-shaped (hidden 4096, MHA 32 x 128,
    # MLP 11008, vocab 32000), cfg2 ranks int8 K, V rank 1640 int4 group-64
    ("cfg5_layers", 2, 4096, 32, 32, 11008, 32000, None, 1640, "int8_g64", 2, 256, 3),
]


@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_e2e_attention_matches_oracle(shape):
    import starkv.e2e as e2e
    name, L, hid, H, Hkv, mlp, vocab, ranks, Rv, fmt, B, P, steps = shape
    ranks = ranks or cfg2_ranks()
    _flush(f"[e2e] {name}: layers={L} hidden={hid} heads={H}/{Hkv} fmt={fmt} B={B} prompt={P} steps={steps}")
    kw = dict(n_layers=L, hidden=hid, heads=H, kv_heads=Hkv, intermediate=mlp, vocab=vocab, ranks=ranks,
              v_rank=Rv, batch=B, capacity=P + steps + 1, fmt=fmt, seed=3)
    g = torch.Generator(device="cuda").manual_seed(5)
    prompt = torch.randint(0, vocab, (B, P), generator=g, device="cuda")
    model = e2e.build_model(**kw)
    with KernelRecorder(e2e) as rec:
        toks, logits = e2e.generate(model, prompt, steps)
    assert [c["kind"] for c in rec.calls] == ["prefill"] * L + ["decode"] * (L * steps)
    assert rec.check() == L * (steps + 1)
    assert all(torch.isfinite(x).all() for x in logits)


@pytest.mark.parametrize("fmt", ["int8_g64", "dense"])
def test_e2e_graph_replay_matches_eager(fmt):
    """Decode steps replayed from one captured graph (device-side cache
    position, masked full-capacity attention) against the same model decoding
    eagerly on the kernels, fed the same tokens: every replay's logits within
    mean-rel 1e-3 of the eager step's (the same kernels over the same
    latents), the greedy tokens equal."""
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
    _compare_logits(logits, ref_logits, tol=1e-3)
    assert torch.equal(toks, ref_toks)
    assert all(layer.self_attn.cache.length == P + steps for layer in model.model.layers)


@pytest.mark.gpu
def test_fused_layers_follow_loaded_weights():
    """fuse_layers_ packs decode copies of each layer's weights (norms folded
    in) and of the output projection; weights loaded afterwards
    (load_state_dict, written in place) must reach them: a model built with
    one seed that loads another seed's state decodes like a model built with
    that seed."""
    from starkv.e2e import build_model, generate
    _flush("[e2e] fused layers after load_state_dict")
    B, P, steps = 2, 24, 4
    kw = dict(n_layers=2, hidden=1024, heads=8, kv_heads=2, intermediate=2048, vocab=1000, ranks=[48, 96],
              v_rank=256, batch=B, capacity=P + steps + 3, fmt="int8_g64")
    prompt = torch.randint(0, 1000, (B, P), generator=torch.Generator(device="cuda").manual_seed(8), device="cuda")
    want = build_model(seed=5, **kw)
    toks, logits = generate(want, prompt, steps)
    model = build_model(seed=4, **kw)
    model.load_state_dict(want.state_dict())
    got_toks, got = generate(model, prompt, steps, forced=toks[:, :steps])
    torch.cuda.synchronize()
    _compare_logits(got, logits, tol=1e-3)
    assert torch.equal(got_toks, toks)


@pytest.mark.gpu
def test_fused_layers_keep_recorded_hidden_states():
    """The fused decoder layer updates the residual stream in place; with
    output_hidden_states=True HF keeps every layer's output, so those must
    survive the layers after them: each recorded hidden state matches the
    reference path's (HF's own layers over the same latent attention)."""
    from starkv.e2e import attention_layers, build_model
    _flush("[e2e] output_hidden_states through the fused layers")
    B, P = 2, 24
    kw = dict(n_layers=3, hidden=1024, heads=8, kv_heads=2, intermediate=2048, vocab=1000, ranks=[48, 96],
              v_rank=256, batch=B, capacity=P + 4, fmt="int8_g64", seed=6)
    prompt = torch.randint(0, 1000, (B, P), generator=torch.Generator(device="cuda").manual_seed(9), device="cuda")
    pos = torch.arange(P, device="cuda")[None].expand(B, P)
    outs = []
    for reference in (False, True):
        model = build_model(**kw)
        for att in attention_layers(model):
            att.reference = reference
        model.model.norm.starkv_reference = reference
        with torch.no_grad():
            outs.append(model(input_ids=prompt, position_ids=pos, use_cache=False, output_hidden_states=True))
    torch.cuda.synchronize()
    got, ref = outs[0].hidden_states, outs[1].hidden_states
    assert len(got) == len(ref) == kw["n_layers"] + 1
    for i, (g, r) in enumerate(zip(got, ref)):
        mx, mr = errors(g.float(), r.float())
        _flush(f"   hidden state {i}: max_abs={mx:.3e} mean_rel={mr:.3e}")
        assert mr <= 1e-2, (i, mr)
    assert not torch.equal(got[1], got[-1])


def test_e2e_graph_state_reports_a_skipped_row():
    """The graph state's error flag, set by a kernel that skipped a row at a
    run-time position outside its table (forced from the host: the device
    position is set past it), makes ``check`` raise."""
    from starkv import RopeConfig, StarKVError, rope_apply
    from starkv.e2e import DecodeGraphState
    from starkv.rope import rope_table
    state = DecodeGraphState(2, 8, 8, "cuda")
    state.check()                                      # nothing skipped yet
    _, cap = rope_table(RopeConfig(), 8, "cuda")
    state.pos.fill_(cap)
    q = torch.zeros(2, 4, 1, 128, device="cuda").half()
    rope_apply(q, RopeConfig(), pos0_device=state.pos, max_positions=8, error_flag=state.error)
    with pytest.raises(StarKVError, match="capacity"):
        state.check()


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
    padded to multiples of 8): every attention call against the oracle."""
    import starkv.e2e as e2e
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
    model = e2e.build_model(**kw)
    with KernelRecorder(e2e) as rec:
        toks, logits = e2e.generate(model, prompt, steps)
    assert rec.check() == 2 * (steps + 1)
    assert all(torch.isfinite(x).all() for x in logits)


def test_e2e_graphed_decode_cfg5_layer_matches_oracle():
    """The path the e2e tok/s times: decode steps replayed from one captured
    graph, each attention over the whole cache capacity with the positions
    after the device-held write position at -1e30, at the e2e workload's layer
    shape (hidden 4096, MHA 32 x 128, cfg2 ranks int8 K, V rank 1640 int4
    group-64) with capacity past the length.  Every layer's attention output
    of every step -- the eager first step and each replay, whose recorded
    buffers the replay rewrites -- is checked against the fp64 oracle over
    the caches as they stand after that step."""
    import starkv.e2e as e2e
    L, B, P, steps = 2, 2, 200, 4
    cap = P + steps + 5
    _flush(f"[e2e graphed cfg5 layers] layers={L} B={B} prompt={P} steps={steps} capacity={cap}")
    model = e2e.build_model(n_layers=L, hidden=4096, heads=32, kv_heads=32, intermediate=11008, vocab=32000,
                            ranks=cfg2_ranks(), v_rank=1640, batch=B, capacity=cap, fmt="int8_g64", seed=7)
    prompt = torch.randint(0, 32000, (B, P), generator=torch.Generator(device="cuda").manual_seed(8), device="cuda")
    checked = []
    with torch.no_grad():
        out = model(input_ids=prompt, position_ids=torch.arange(P, device="cuda")[None].expand(B, P),
                    use_cache=False, logits_to_keep=1)
        tok = out.logits[:, -1].argmax(-1, keepdim=True)
        with KernelRecorder(e2e) as rec:
            def on_step(i):
                calls = rec.calls[-L:]
                assert len(calls) == L and all(c["kind"] == "decode" and c["S"] == cap and int(c["last_pos"].reshape(-1)[0]) == P + i
                                               for c in calls)
                view = KernelRecorder(e2e)
                view.calls = calls
                _flush(f"   step {i} ({'eager' if i == 0 else 'replay'}), position {P + i}")
                checked.append(view.check())
            toks, _ = e2e.decode_graphed(model, tok, steps, keep_logits=False, on_step=on_step)
    assert toks.shape == (B, steps)
    assert checked == [L] * steps
    assert all(layer.self_attn.cache.length == P + steps for layer in model.model.layers)
