"""Benchmark of the STAR-KV fused decode-attention path on one MI355X.

Workload (the metric's configuration, "cfg2"): Llama-2-7B-shaped layer, MHA
32 heads x 128, fp16, batch 16, context 32768, head-wise K ranks from
{16..96} (sum 1640, committed fixture), V rank 1640, one decode query token.
Synthetic seeded data, inputs resident in HBM before timing.

A "step" is one decode-attention pass of one layer over the whole batch:
K-logits (latent K reconstruction + RoPE + q.K), softmax, P.V latent and the
B_v up-projection -- the scope of the reference's "attention us/layer"
(latency.py:262-268).

Prints ONE JSON line.  value = algorithmic HBM bytes of the step / step time
(GB/s); roofline = the dominant kernel against MI355X's 8 TB/s HBM;
cpu_baseline = the reference's eager PyTorch decode path restated op for op
(oracle/starkv_oracle.py), timed on this host's cores at config 1 (the
CPU-baseline layer), with the same restatement on batch 1 of the cfg2
workload as an extra key.  The default run then measures the metric's second
half, e2e decode tok/s (the e2e workload below), and adds it to the line
(``e2e_decode_tok_s`` and ``e2e``; ``--no-e2e`` skips it).
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "star-kv_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
HEAD_DIM = 128


def algorithmic_bytes(case):
    """Per-step algorithmic bytes: latent caches + B_k + U_v + q + output."""
    esz = 2
    xk = sum(case.B * case.S * r for r in case.ranks) * esz
    xv = case.B * case.S * case.Rv * esz
    bk = sum(case.ranks) * HEAD_DIM * esz
    uv = case.Hkv * HEAD_DIM * case.Rv * esz
    q = case.B * case.Hq * HEAD_DIM * esz
    out = case.B * case.Hq * HEAD_DIM * esz
    return {"k_logits": xk + bk + q, "pv_latent": xv, "up_proj": uv + out, "total": xk + xv + bk + uv + q + out}


def cpu_baseline(case_cpu_fn, reps, warmup=3, min_reps=20, budget_s=15.0):
    """Time the oracle's eager restatement of the reference decode path on
    this host's cores: ``warmup`` untimed calls, then at least ``min_reps``
    timed ones (more while the time budget lasts, up to ``reps``); returns
    (median seconds, os.cpu_count(), torch.get_num_threads(), reps timed)."""
    import torch
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    fn = case_cpu_fn()
    for _ in range(warmup):
        fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    for _ in range(max(reps, min_reps)):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if len(ts) >= min_reps and time.perf_counter() > t_end:
            break
    return statistics.median(ts), threads, torch.get_num_threads(), len(ts)


def cfg1_inputs():
    """Config 1, the CPU-baseline layer: batch 1, 32
    heads x 128, context 1024, K rank 32 per head, V rank 1024, fp32, seed 0.
    Latents and q ~N(0,1), B_k [32 x 128] per head ~N(0,1/32), B_v
    [1024 x 4096] ~N(0,1/1024) (U_v = v_proj.U.weight = B_v^T), theta 10000.
    Returns the oracle's decode arguments and the algorithmic bytes."""
    import torch
    from oracle import starkv_oracle as o
    g = torch.Generator().manual_seed(0)
    B, H, S, r, Rv = 1, 32, 1024, 32, 1024
    q = torch.randn(B, H, HEAD_DIM, generator=g)
    xk = [torch.randn(B, S, r, generator=g) for _ in range(H)]
    bk = [torch.randn(r, HEAD_DIM, generator=g) / math.sqrt(r) for _ in range(H)]
    xv = torch.randn(B, S, Rv, generator=g)
    bv = torch.randn(Rv, H * HEAD_DIM, generator=g) / math.sqrt(Rv)
    uv = bv.t().contiguous()
    cos, sin = o.rope_cos_sin(o.rope_inv_freq(10000.0), torch.arange(S))
    nbytes = 4 * (B * S * H * r + B * S * Rv + H * r * HEAD_DIM + Rv * H * HEAD_DIM + 2 * B * H * HEAD_DIM)
    return (q, bk, xk, xv, uv, cos, sin), nbytes


def cfg1_cpu_baseline(reps):
    """The reference's eager decode path (abx_rope_batched.py:189-202 with
    per-position RoPE, model.py:458-487) restated op for op by the oracle,
    fp32 on this host, at config 1."""
    import torch
    from oracle import starkv_oracle as o
    args, nbytes = cfg1_inputs()

    def make_fn():
        def fn():
            with torch.no_grad():
                o.decode_attention(*args, dtype=torch.float32)
        return fn

    med, cores, nthreads, n = cpu_baseline(make_fn, reps)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
            "host_cpus": cores, "torch_threads": nthreads, "us_per_layer": round(med * 1e6, 1),
            "sample": f"config 1 (B1, 32 heads x 128, S1024, K rank 32/head, V rank 1024, fp32, seed 0): the "
                      f"reference eager decode path restated op for op (oracle.starkv_oracle.decode_attention: "
                      f"X_k B_k, per-position RoPE, q K^T / sqrt(128), fp32 softmax, P X_v, U_v), 3 warm-ups, "
                      f"median of {n} reps; value = algorithmic bytes ({nbytes}) / median time"}


def build_workload(name, dev):
    """Seeded synthetic inputs of one workload, resident in HBM; returns the
    step function and the algorithmic bytes per step."""
    import torch
    from _util import cfg2_ranks, cfg4_ranks, make_case
    from starkv import RopeConfig, VLatentSpec, decode_attention
    from starkv.cache import LatentCache

    if name == "cfg2":
        ranks = cfg2_ranks()
        B, H, S, Rv = 16, 32, 32768, 1640
        case = make_case(B, H, H, S, ranks, Rv, dtype=torch.float16, device=dev, seed=0)
        rope = RopeConfig()
        out = torch.empty(B, H, HEAD_DIM, dtype=torch.float16, device=dev)

        def step(ev=None):
            decode_attention(case.q, case.kspec, case.xv, case.uv, rope=rope, out=out, events=ev)
        cfg = {"workload": "cfg2: Llama-2-7B-shaped decode attention layer, MHA 32x128, fp16, batch 16, "
                           "context 32768, ragged K ranks (sum 1640), V rank 1640",
               "batch": B, "seq_len": S, "k_rank_total": sum(ranks), "v_rank": Rv, "heads": H}
        return dict(case=case, bytes=algorithmic_bytes(case), step=step, B=B, S=S, rope=rope, dtype="f16", config=cfg)

    if name in ("cfg3", "cfg3-long", "cfg3-e2e", "cfg3-e2e-mask"):
        ranks = cfg2_ranks()
        # cfg3-e2e: the e2e harness's attention shape (B8, prompt 8192 + 256
        # decode steps + 1 of cache capacity)
        # cfg3-e2e-mask: the same under the harness's additive device mask
        # ([B, 1, S] fp32, -1e30 on the positions not yet written)
        B, S = {"cfg3": (16, 32768), "cfg3-long": (4, 131072), "cfg3-e2e": (8, 8449),
                "cfg3-e2e-mask": (8, 8449)}[name]
        H, Rv, rmax = len(ranks), 1640, max(ranks)
        g = torch.Generator(device=dev).manual_seed(0)
        k_new = torch.randn(B, H, S, rmax, generator=g, device=dev, dtype=torch.float16)
        k_new[..., ::97] *= 10                                   # 1 % outlier channels
        v_new = torch.randn(B, S, Rv, generator=g, device=dev, dtype=torch.float16)
        v_new[..., ::97] *= 10
        bk = (torch.randn(H, rmax, HEAD_DIM, generator=g, device=dev) / math.sqrt(rmax)).half()
        uv = (torch.randn(H * HEAD_DIM, Rv, generator=g, device=dev) / math.sqrt(Rv)).half()
        q = torch.randn(B, H, HEAD_DIM, generator=g, device=dev).half()
        cache = LatentCache(B, ranks, Rv, S, torch.float16, dev, fmt="int8_g64")
        kspec, vspec, _ = cache.append(k_new, v_new, bk)
        del k_new, v_new
        torch.cuda.empty_cache()
        rope = RopeConfig()
        out = torch.empty(B, H, HEAD_DIM, dtype=torch.float16, device=dev)
        mask = None
        if name == "cfg3-e2e-mask":
            mask = torch.zeros(B, 1, S, dtype=torch.float32, device=dev)
            mask[:, :, S - 128:] = -1e30

        def step(ev=None):
            decode_attention(q, kspec, vspec, uv, rope=rope, seq_len=S, out=out, events=ev, mask=mask)
        G = (Rv + 63) // 64
        xk = B * S * sum(ranks) + B * H * S * 2                  # int8 + fp16 scale per (b, h, s)
        xv = B * S * Rv // 2 + B * S * G * 4                     # packed int4 + fp16 scale and zero per group
        w = sum(ranks) * HEAD_DIM * 2 + H * HEAD_DIM * Rv * 2
        qo = 2 * B * H * HEAD_DIM * 2
        nb = {"k_logits": xk + sum(ranks) * HEAD_DIM * 2 + B * H * HEAD_DIM * 2, "pv_latent": xv,
              "up_proj": H * HEAD_DIM * Rv * 2 + B * H * HEAD_DIM * 2, "total": xk + xv + w + qo}
        cfg = {"workload": f"{name}: Llama-2-7B-shaped layer, fp16, batch {B}, context {S}, ragged K ranks "
                           f"(sum 1640) int8 with fp16 scale per (b,h,s), V rank 1640 int4 asymmetric g64 "
                           f"(fp16 scale+zero), 1 % outlier channels",
               "batch": B, "seq_len": S, "k_rank_total": sum(ranks), "v_rank": Rv, "heads": H}
        return dict(case=None, bytes=nb, step=step, B=B, S=S, rope=rope, dtype="f16", config=cfg)

    if name.startswith("cfg4-"):
        S = int(name.split("-", 1)[1])
        ranks = cfg4_ranks()
        B, Hq, Hkv, Rv = 1, 32, 8, 512
        rope = RopeConfig(theta=500000.0, rope_type="llama3", factor=8.0, low_freq_factor=1.0,
                          high_freq_factor=4.0, original_max_position_embeddings=8192)
        G = (Rv + 63) // 64
        xk = B * S * sum(ranks) * 2
        xv = B * S * Rv // 2 + B * S * G * 4
        nb = {"k_logits": xk + sum(ranks) * HEAD_DIM * 2 + B * Hq * HEAD_DIM * 2, "pv_latent": xv,
              "up_proj": Hkv * HEAD_DIM * Rv * 2 + B * Hq * HEAD_DIM * 2,
              "total": xk + xv + sum(ranks) * HEAD_DIM * 2 + Hkv * HEAD_DIM * Rv * 2 + 2 * B * Hq * HEAD_DIM * 2}
        # the whole working set of one step is ~0.2 GB at S=131072 and less below,
        # inside the 256 MB MALL: steps rotate over copies of every input (latents,
        # scales, weights, q) that together span >= 512 MB, so each step streams
        # its bytes from HBM
        n_copies = max(1, min(1024, -(-(512 << 20) // nb["total"])))
        copies = []
        g = torch.Generator(device=dev).manual_seed(6)
        for c in range(n_copies):
            case = make_case(B, Hq, Hkv, S, ranks, Rv, dtype=torch.bfloat16, device=dev, seed=5 + c)
            vp = torch.randint(0, 256, (B, S, Rv // 2), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
            vs = (torch.rand(B, S, G, generator=g, device=dev) * 0.3 + 0.05).half()
            vz = (-torch.rand(B, S, G, generator=g, device=dev) * 2).half()
            copies.append((case, VLatentSpec.int4_g64(vp, vs, vz, Rv)))
        case = copies[0][0]
        out = torch.empty(B, Hq, HEAD_DIM, dtype=torch.bfloat16, device=dev)
        turn = [0]

        def step(ev=None):
            c, vspec = copies[turn[0] % n_copies]
            turn[0] += 1
            decode_attention(c.q, c.kspec, vspec, c.uv, rope=rope, out=out, events=ev)
        cfg = {"workload": f"{name}: Llama-3.1-8B-shaped GQA layer (32 q / 8 KV heads, llama3 RoPE theta 500000), "
                           f"bf16, batch 1, context {S}, K ranks per KV head in [32,128] (bf16), V rank 512 int4 "
                           f"asymmetric g64",
               "batch": B, "seq_len": S, "k_rank_total": sum(ranks), "v_rank": Rv, "heads": Hq, "kv_heads": Hkv,
               "rotated_input_copies": n_copies}
        return dict(case=case, bytes=nb, step=step, B=B, S=S, rope=rope, dtype="bf16", config=cfg)
    if name.startswith("abx-"):
        # the reference's abx benchmark (abx_rope_batched.py:205-250, 274-280):
        # total rank int(0.2 * 4096) = 819 over 32 query heads in KV groups of
        # 4 -> 8 KV heads of rank 102, fp16, theta 10000, one query per head,
        # at a context from target_seq_lens (4096, 16384, 65536, 262144); its
        # tensors carry no batch dimension, i.e. batch 1.  A step is one abx
        # call (the K-logit kernel): fp16 logits [1, 32, 1, S] out.
        from starkv.abx_rope_batched import abx
        S = int(name.split("-", 1)[1])
        B, Hq, Hkv = 1, 32, 8
        r = int(4096 * 0.2) // Hkv
        per = {"x": B * Hkv * S * r * 2, "b": Hkv * r * HEAD_DIM * 2, "a": B * Hq * HEAD_DIM * 2, "out": B * Hq * S * 2}
        tot = sum(per.values())
        nb = {"k_logits": tot, "pv_latent": 0, "up_proj": 0, "total": tot}
        # rotate over input copies spanning >= 512 MB so each call streams from HBM
        n_copies = max(1, min(1024, -(-(512 << 20) // tot)))
        g = torch.Generator(device=dev).manual_seed(7)
        copies = [(torch.randn(B, Hq, 1, HEAD_DIM, generator=g, device=dev).half(),
                   (torch.randn(Hq, r, HEAD_DIM, generator=g, device=dev) / math.sqrt(r)).half(),
                   torch.randn(B, Hkv, S, r, generator=g, device=dev).half()) for _ in range(n_copies)]
        turn = [0]

        def step(ev=None):
            a, b, x = copies[turn[0] % n_copies]
            turn[0] += 1
            if ev:
                ev[0].record()
            abx(a, b, x, dtype=torch.float16)
            if ev:
                for e in ev[1:]:
                    e.record()
        cfg = {"workload": f"{name}: the reference's abx micro-benchmark shape (abx_rope_batched.py:274-280): "
                           f"32 query heads in KV groups of 4, 8 KV heads of K rank 102 (total 819), fp16, "
                           f"batch 1, context {S}; one abx call (K logits with RoPE, fp16 out)",
               "batch": B, "seq_len": S, "k_rank_total": Hkv * r, "heads": Hq, "kv_heads": Hkv,
               "rotated_input_copies": n_copies}
        return dict(case=None, bytes=nb, step=step, B=B, S=S, rope=RopeConfig(), dtype="f16", config=cfg)
    raise SystemExit(f"unknown workload {name!r}")


def graphed_attention_ms(atts, B, reps=20):
    """The attention work of one graph-replayed decode step on its own: for
    every layer the cache write with the query rotation (one launch) and the
    decode attention over the whole cache capacity, positions past the
    device-held write position at -1e30 --
    the calls LatentAttention.core makes in the captured step, on the same
    caches at the same length -- captured in one graph of their own and
    replayed; returns ms per replay.  (Each replay rewrites the first free
    cache position, which no real step has written yet.)"""
    import torch
    from starkv import decode_attention
    from starkv.e2e import DecodeGraphState
    a0 = atts[0]
    dev = a0.bk.device
    L, cap = a0.cache.length, a0.cache.cap
    assert L < cap, "the attention-only graph writes one free cache position"
    state = DecodeGraphState(B, cap, L, dev)
    g = torch.Generator(device=dev).manual_seed(11)
    bufs = [(torch.randn(B, a.n_heads, 1, HEAD_DIM, generator=g, device=dev).half(),
             torch.randn(B, 1, sum(a.ranks), generator=g, device=dev).half(),
             torch.randn(B, 1, a.v_u.weight.shape[1], generator=g, device=dev).half()) for a in atts]

    def attn():
        for a, (q, k, v) in zip(atts, bufs):
            ks, vs = a.cache.append_at(k, v, a.bk, state.pos, error_flag=state.error, q=q, rope=a.rope)
            decode_attention(q[:, :, 0], ks, vs, a.v_u.weight, rope=a.rope, seq_len=state.capacity,
                             scale=a.scaling, last_pos=state.pos)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        attn()                                        # eager once: tables and workspace in place
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        attn()
    for _ in range(3):
        graph.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    state.check()
    return e0.elapsed_time(e1) / reps


def run_e2e(args, emit=True):
    """End-to-end decode (the e2e configuration): random-init 32-layer
    Llama-2-7B-shaped model (vocab 32000, MLP 11008, fp16), every attention on
    the latent cache (cfg3 ranks and formats: K int8, V int4-g64), prefill 8192
    random tokens at batch 8 (starkv_prefill_attention), then greedy decode
    steps replayed from one captured HIP graph (starkv.e2e.decode_graphed).
    The attention share is the attention work of one step, captured and
    replayed as a graph of its own (graphed_attention_ms), over the timed
    step."""
    import torch
    from _util import cfg2_ranks
    from starkv.e2e import attention_layers, build_model, decode_graphed
    B, P, steps = 8, 8192, args.e2e_steps
    t0 = time.perf_counter()
    model = build_model(n_layers=32, hidden=4096, heads=32, kv_heads=32, intermediate=11008, vocab=32000,
                        ranks=cfg2_ranks(), v_rank=1640, batch=B, capacity=P + steps + 1,
                        fmt="int8_g64", seed=0)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    g = torch.Generator(device="cuda").manual_seed(0)
    prompt = torch.randint(0, 32000, (B, P), generator=g, device="cuda")
    atts = attention_layers(model)
    with torch.no_grad():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = model(input_ids=prompt, position_ids=torch.arange(P, device="cuda")[None].expand(B, P),
                    use_cache=False, logits_to_keep=1)
        tok = out.logits[:, -1].argmax(-1, keepdim=True)
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        # graph-replayed decode: the timed region
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks, _ = decode_graphed(model, tok, steps, keep_logits=False)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        # the same step's attention work alone, graph-replayed, at the context
        # the decode ended on
        attn_ms = graphed_attention_ms(atts, B)
    step_s = wall / steps
    n_layers = len(atts)
    rec = {
        "metric": "e2e decode tok/s", "value": round(B * steps / wall, 1), "unit": "tok/s", "n_gpus": 1,
        "steps": steps, "higher_is_better": True, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "e2e: random-init 32-layer Llama-2-7B-shaped model (vocab 32000, MLP 11008, fp16), "
                               "every attention on a STAR-KV latent cache (ragged K ranks sum 1640 int8, V rank 1640 "
                               "int4-g64), prefill 8192 random tokens, greedy decode at batch 8 replayed from one "
                               "captured HIP graph",
                   "batch": B, "prompt": P, "decode_steps": steps},
        "ms_per_decode_step": round(step_s * 1e3, 3),
        # every layer's cache write + query rotation and decode attention of
        # one step, captured and replayed as a graph of their own (context
        # P + steps), against the timed graph-replayed step
        "attention_ms_per_decode_step": round(attn_ms, 3),
        "attention_us_per_layer": round(attn_ms * 1e3 / n_layers, 1),
        "attention_share": round(attn_ms / (step_s * 1e3), 4),
        "prefill_s": round(t_prefill, 3), "build_s": round(t_build, 1),
    }
    del model
    if emit:
        print(json.dumps(rec), flush=True)
    return rec


MFMA_PEAK_TFLOPS = 2500.0     # MI355X dense fp16 / bf16 MFMA


def prefill_flops(B, Hq, Hkv, T, pos0, ranks, Rv):
    """Algorithmic FLOPs of one causal prefill layer: K reconstruction
    2*B*S*sum(r)*128, V reconstruction 2*B*S*Rv*Hkv*128 (S = pos0 + T), and
    the attention 4*128 per visible (query, key) pair per query head (q.K and
    P.V), sum over t of pos0 + t + 1 visible keys."""
    S = pos0 + T
    recon_k = 2 * B * S * sum(ranks) * HEAD_DIM
    recon_v = 2 * B * S * Rv * Hkv * HEAD_DIM
    pairs = T * pos0 + T * (T + 1) // 2
    attn = 4 * HEAD_DIM * B * Hq * pairs
    return {"recon": recon_k + recon_v, "attention": attn, "total": recon_k + recon_v + attn}


def run_prefill(args):
    """Prefill of one attention layer: the 8192-token prompt at batch 8 of the
    e2e workload (Llama-2-7B-shaped MHA 32 x 128, fp16, ragged K ranks sum 1640
    as int8, V rank 1640 as int4-g64).  A step is starkv_prefill_attention:
    K / V reconstruction from the latents + causal flash attention."""
    import torch
    from _util import cfg2_ranks
    from starkv import RopeConfig, prefill_attention
    from starkv.cache import LatentCache
    B, T, Hq, Rv = 8, 8192, 32, 1640
    ranks = cfg2_ranks()
    Hkv = len(ranks)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    rmax = max(ranks)
    bk = torch.zeros(Hkv, rmax, HEAD_DIM, device=dev)
    k_new = torch.zeros(B, Hkv, T, rmax, device=dev, dtype=torch.float16)
    for h, r in enumerate(ranks):
        bk[h, :r] = torch.randn(r, HEAD_DIM, generator=g, device=dev) / math.sqrt(r)
        k_new[:, h, :, :r] = torch.randn(B, T, r, generator=g, device=dev).half()
    bk = bk.half()
    v_new = torch.randn(B, T, Rv, generator=g, device=dev).half()
    cache = LatentCache(B, ranks, Rv, T, torch.float16, dev, fmt="int8_g64")
    kspec, vspec, S = cache.append(k_new, v_new, bk)
    del k_new, v_new
    uv = (torch.randn(Hkv * HEAD_DIM, Rv, generator=g, device=dev) / math.sqrt(Rv)).half()
    q = torch.randn(B, Hq, T, HEAD_DIM, generator=g, device=dev).half()
    out = torch.empty_like(q)
    rope = RopeConfig()
    fl = prefill_flops(B, Hq, Hkv, T, 0, ranks, Rv)

    def step(ev=None):
        prefill_attention(q, kspec, vspec, uv, rope=rope, out=out, events=ev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for e3 in evs:
        for e in e3:
            e.record()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    rec_ms = statistics.mean([e[0].elapsed_time(e[1]) for e in evs])
    fa_ms = statistics.mean([e[1].elapsed_time(e[2]) for e in evs])
    ms = statistics.mean([e[0].elapsed_time(e[2]) for e in evs])
    tflops = fl["total"] / (ms * 1e-3) / 1e12
    fa_tflops = fl["attention"] / (fa_ms * 1e-3) / 1e12

    # the reference's own prefill route on this GPU (model.py:429-449: K / V
    # materialised by torch matmuls from the dequantised latents, RoPE, GQA
    # repeat, SDPA with the causal mask), timed for comparison
    torch_ms = None
    try:
        if args.no_torch_reference:
            raise torch.cuda.OutOfMemoryError("skipped")
        xk = cache.dequant_k(S)
        xv = cache.dequant_v(S)
        cos, sin = rope.cos_sin(torch.arange(S, device=dev))
        cos, sin = cos.half(), sin.half()

        def torch_step():
            ks = []
            for h in range(Hkv):
                kh = torch.matmul(xk[h], bk[h, :ranks[h]])
                ks.append(kh * cos + torch.cat((-kh[..., 64:], kh[..., :64]), -1) * sin)
            K = torch.stack(ks, 1)
            V = torch.nn.functional.linear(xv, uv).view(B, S, Hkv, HEAD_DIM).transpose(1, 2)
            return torch.nn.functional.scaled_dot_product_attention(q, K, V.contiguous(), is_causal=True)

        for _ in range(2):
            torch_step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        n_t = max(1, min(5, args.steps))
        for _ in range(n_t):
            torch_step()
        torch.cuda.synchronize()
        torch_ms = (time.perf_counter() - t1) * 1e3 / n_t
        del xk, xv
    except torch.cuda.OutOfMemoryError:
        torch_ms = None

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import starkv_oracle as o
        Ts = 4096

        def make_fn():
            xk1 = [cache.dequant_k(Ts)[0][:1].float().cpu()]
            xv1 = cache.dequant_v(Ts)[:1].float().cpu()
            c = dict(q=q[:1, :1, :Ts].float().cpu(), bk=[bk[0, :ranks[0]].float().cpu()], xk=xk1, xv=xv1,
                     uv=uv[:HEAD_DIM].float().cpu())
            cs, sn = o.rope_cos_sin(rope.inv_freq(), torch.arange(Ts), 1.0)

            def fn():
                with torch.no_grad():
                    o.prefill_attention(c["q"], c["bk"], c["xk"], c["xv"], c["uv"], cs, sn, dtype=torch.float32)
            return fn

        med, cores, nthreads, n = cpu_baseline(make_fn, args.cpu_reps)
        sfl = prefill_flops(1, 1, 1, Ts, 0, ranks[:1], Rv)["total"]
        cpu = {"value": round(sfl / med / 1e12, 5), "unit": "TFLOP/s", "cores": nthreads, "kind": "port",
               "host_cpus": cores, "ms_per_sample": round(med * 1e3, 1),
               "sample": f"batch 1, query head 0 (KV head 0, rank {ranks[0]}), {Ts} tokens, fp32 torch eager "
                         f"restatement of the reference prefill (oracle.starkv_oracle.prefill_attention, causal), "
                         f"median of {n} reps; FLOPs counted as for the GPU line"}

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_prefill.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("fa_causal")
    rec = {
        "metric": "prefill attention TFLOP/s per layer (MFMA roofline)",
        "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "prefill: one Llama-2-7B-shaped layer (MHA 32 x 128, fp16), batch 8, 8192-token "
                               "causal prompt over a latent cache (ragged K ranks sum 1640 int8, V rank 1640 "
                               "int4-g64) -- the e2e workload's prefill",
                   "batch": B, "tokens": T, "k_ranks_sum": sum(ranks), "v_rank": Rv},
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
        "prefill_tokens_per_s": round(B * T / (ms * 1e-3), 1),
        "kernels_ms": {"kv_recon": round(rec_ms, 4), "fa_causal": round(fa_ms, 4)},
        "algorithmic_flops": fl,
        "torch_reference_gpu_ms": round(torch_ms, 3) if torch_ms else None,
        "roofline": {"bound": "mfma", "kernel": "fa_causal", "achieved": round(fa_tflops, 1),
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(fa_tflops / MFMA_PEAK_TFLOPS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-torch-reference", action="store_true",
                    help="skip timing the reference's eager torch decode route on the GPU (cfg2)")
    ap.add_argument("--cpu-reps", type=int, default=100)
    ap.add_argument("--workload", default="cfg2",
                    help="cfg2 (default: the metric's workload), cfg3 (B16 S32768, K int8 + V int4-g64 cache), "
                         "cfg3-long (B4 S131072, same formats), cfg3-e2e (B8 S8449, the e2e attention shape), cfg4-<S> (llama3 GQA bf16 B1, V int4-g64, context S), "
                         "abx-<S> (the reference's abx micro-benchmark: 8 KV heads of rank 102, groups of 4, fp16, batch 1), "
                         "e2e (32-layer model, prefill 8192, greedy decode at batch 8; prints e2e decode tok/s), "
                         "prefill (one layer's 8192-token causal prefill at batch 8 over the int8 / int4-g64 "
                         "latent cache; prints TFLOP/s against the MFMA roofline)")
    ap.add_argument("--e2e-steps", type=int, default=256)
    ap.add_argument("--no-e2e", action="store_true",
                    help="default workload: skip the e2e decode measurement that follows the layer measurement")
    ap.add_argument("--pmc-calibrate", action="store_true",
                    help="only run three 1 GiB device-to-device copies (the known-size reference for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE per dispatch) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "e2e":
        run_e2e(args)
        return
    if args.workload == "prefill":
        run_prefill(args)
        return
    if args.pmc_calibrate:
        n = 1 << 30
        src = torch.full((n // 4,), 7, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes_read": n, "calibration_copy_bytes_written": n, "copies": 3}))
        return
    wl = build_workload(args.workload, dev)
    case, nbytes, step, B, S = wl["case"], wl["bytes"], wl["step"], wl["B"], wl["S"]
    rope = wl["rope"]

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # timed region: the K steps captured in one HIP graph and replayed once,
    # HIP events only at its two ends.  Launched one by one from Python, a
    # small shape's step would measure the host's launch rate, and events
    # between the kernels add a few us of their own.  Workloads that rotate
    # over input copies (to stream from HBM, not the 256 MB MALL) write
    # 512 MB between the warm-up replay and the timed one, so the timed
    # replay does not find the warm-up's copies cached.
    timing = "hip_graph"
    graph = None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(args.steps):
                step()
        graph.replay()
        torch.cuda.synchronize()
    except Exception as e:                       # capture refused: time the steps as launched
        graph = None
        timing = f"eager ({type(e).__name__})"
        torch.cuda.synchronize()
    flush = None
    if wl["config"].get("rotated_input_copies"):
        flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        flush.zero_()
    t_beg, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    t_beg.record()
    if graph is not None:
        graph.replay()
    else:
        for i in range(args.steps):
            step()
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = t_beg.elapsed_time(t_end) / args.steps
    del graph, flush
    # per-kernel breakdown: the same steps again with events between the
    # three kernels (their durations include the events' own gaps)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    for e4 in evs:
        for e in e4:
            e.record()
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    k1 = [e[0].elapsed_time(e[1]) for e in evs]
    k2 = [e[1].elapsed_time(e[2]) for e in evs]
    k3 = [e[2].elapsed_time(e[3]) for e in evs]
    step_ev_ms = statistics.mean([e[0].elapsed_time(e[3]) for e in evs])
    wall_ms = wall * 1e3 / args.steps
    ms = max(gpu_ms, 1e-9)
    k1m, k2m, k3m = statistics.mean(k1), statistics.mean(k2), statistics.mean(k3)
    gbs = nbytes["total"] / (ms * 1e-3) / 1e9

    dom = "k_logits" if k1m >= k2m else "pv_latent"
    dom_ms = k1m if dom == "k_logits" else k2m
    dom_gbs = nbytes[dom] / (dom_ms * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_cfg2.json")
    if args.workload == "cfg2" and os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get(dom)

    # the reference's eager torch decode route on this GPU (model.py:450-487 with
    # torch_abx's per-head reconstruction, abx_rope_batched.py:189-202), timed
    # for comparison: K materialised per KV head, RoPE, q.K, softmax in fp32,
    # P @ X_v, per-head up-projection
    torch_ref_us = None
    if args.workload == "cfg2" and not args.no_torch_reference:
        try:
            cos, sin = rope.cos_sin(torch.arange(S, device=dev))
            cos, sin = cos.half(), sin.half()
            gs = case.Hq // case.Hkv
            U = case.uv.view(case.Hkv, HEAD_DIM, case.Rv)

            def torch_step():
                logits = torch.empty(B, case.Hq, S, dtype=torch.float16, device=dev)
                for h in range(case.Hkv):
                    K = torch.matmul(case.xk_heads[h], case.bk_heads[h])
                    K = K * cos + torch.cat((-K[..., 64:], K[..., :64]), -1) * sin
                    qh = case.q[:, h * gs:(h + 1) * gs].contiguous()
                    logits[:, h * gs:(h + 1) * gs] = torch.matmul(qh, K.transpose(1, 2).contiguous())
                p = torch.softmax(logits.float() / math.sqrt(HEAD_DIM), dim=-1).half()
                o_lat = torch.matmul(p, case.xv)                                   # [B, Hq, Rv]
                Uq = U.repeat_interleave(gs, 0)                                    # [Hq, 128, Rv]
                return torch.matmul(o_lat.transpose(0, 1), Uq.transpose(1, 2).contiguous()).transpose(0, 1)

            for _ in range(2):
                torch_step()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            for _ in range(5):
                torch_step()
            torch.cuda.synchronize()
            torch_ref_us = (time.perf_counter() - t1) * 1e6 / 5
        except torch.cuda.OutOfMemoryError:
            torch_ref_us = None

    cpu = cpu_b1 = None
    if not args.no_cpu_baseline and args.workload == "cfg2":
        from oracle import starkv_oracle as o
        cpu = cfg1_cpu_baseline(10 * args.cpu_reps)      # ~10 ms per rep: about 10 s of CPU work

        def make_fn():
            c = {
                "q": case.q[:1].float().cpu(),
                "bk": [b.float().cpu() for b in case.bk_heads],
                "xk": [x[:1].float().cpu() for x in case.xk_heads],
                "xv": case.xv[:1].float().cpu(),
                "uv": case.uv.float().cpu(),
            }
            cos, sin = o.rope_cos_sin(rope.inv_freq(), torch.arange(S), 1.0)

            def fn():
                with torch.no_grad():
                    o.decode_attention(c["q"], c["bk"], c["xk"], c["xv"], c["uv"], cos, sin, dtype=torch.float32)
            return fn

        med, cores, nthreads, n = cpu_baseline(make_fn, args.cpu_reps)
        cpu_bytes = nbytes["total"] / B
        cpu_b1 = {"value": round(cpu_bytes / med / 1e9, 3), "unit": "GB/s", "cores": nthreads,
               "kind": "port", "host_cpus": cores, "us_per_layer_b1": round(med * 1e6, 1),
               "sample": f"cfg2 workload batch 1 of {B} (S={S}), fp32 torch eager restatement of the reference "
                         f"decode path (oracle.starkv_oracle.decode_attention), median of {n} reps"}

    rec = {
        "metric": "decode attn us/layer + HBM GB/s (% peak) at B16 S32K; e2e decode tok/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": "synthetic",
        "config": wl["config"],
        "us_per_layer": round(ms * 1e3, 1),
        "wall_ms_per_step": round(wall_ms, 4),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 1),
        "attn_layer_tokens_per_s": round(B / (ms * 1e-3), 1),
        "kernels_us": {"k_logits": round(k1m * 1e3, 1), "pv_latent": round(k2m * 1e3, 1), "up_proj": round(k3m * 1e3, 1)},
        "us_per_layer_with_kernel_events": round(step_ev_ms * 1e3, 1),
        "timing": timing,
        "algorithmic_bytes": nbytes,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "torch_reference_gpu_us": round(torch_ref_us, 1) if torch_ref_us else None,
        "cpu_baseline": cpu,
        "cpu_baseline_cfg2_b1": cpu_b1,
    }
    if args.workload == "cfg2" and not args.no_e2e:
        # the metric's second half: e2e decode tok/s (the e2e workload), in the
        # same process after the layer measurement
        del case, wl, step
        import gc
        gc.collect()
        torch.cuda.empty_cache()
        e2e = run_e2e(args, emit=False)
        rec["e2e_decode_tok_s"] = e2e["value"]
        rec["e2e"] = {k: e2e[k] for k in ("ms_per_decode_step", "attention_ms_per_decode_step",
                                          "attention_us_per_layer", "attention_share", "prefill_s", "steps",
                                          "config")}
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
