"""Pins of the CPU oracle (oracle/starkv_oracle.py) — CPU only.

Each oracle function is checked against something other than its own
formula: the RoPE fixtures written with transformers (tests/golden/), a
formulation written independently here (complex exponentials, pure-Python
loops, torch SDPA on materialised K/V), invariants (ragged = zero-padded,
GQA head mapping) and exhaustive integer tables.  The "planted" tests swap a
plausible mistake into the oracle and assert that the pin catches it.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import starkv_oracle as o

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "rope_fixtures.npz"))
D = 128


def _llama3_inv():
    return o.rope_inv_freq(500000.0, rope_type="llama3", factor=8.0, low_freq_factor=1.0,
                           high_freq_factor=4.0, original_max_position_embeddings=8192)


# --------------------------------------------------------------------------
# RoPE tables (HF:models/llama/modeling_llama.py:103-134, HF:modeling_rope_utils.py:640-662)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("tag", ["default", "llama3"])
def test_rope_tables_match_transformers_fixtures(tag):
    inv = o.rope_inv_freq() if tag == "default" else _llama3_inv()
    np.testing.assert_array_equal(inv.numpy(), FIX[f"{tag}_inv_freq"])
    pos = torch.from_numpy(FIX["positions"])
    cos, sin = o.rope_cos_sin(inv, pos, float(FIX[f"{tag}_attention_scaling"]))
    np.testing.assert_allclose(cos.numpy(), FIX[f"{tag}_cos"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(sin.numpy(), FIX[f"{tag}_sin"], rtol=0, atol=2e-6)
    q = torch.from_numpy(FIX[f"{tag}_q"])
    qr = o.apply_rope(q, torch.from_numpy(FIX[f"{tag}_cos"]), torch.from_numpy(FIX[f"{tag}_sin"]))
    np.testing.assert_allclose(qr.numpy(), FIX[f"{tag}_qrot"], rtol=0, atol=1e-6)


def test_rope_closed_forms():
    inv = o.rope_inv_freq()
    assert inv[0].item() == 1.0                              # theta^0
    assert abs(inv[-1].item() - 10000.0 ** (-126 / 128)) < 1e-9
    cos, sin = o.rope_cos_sin(inv, torch.arange(0, 4096, 7))
    torch.testing.assert_close(cos * cos + sin * sin, torch.ones_like(cos), atol=2e-6, rtol=0)
    c0, s0 = o.rope_cos_sin(inv, torch.tensor([0]))
    assert torch.equal(c0, torch.ones_like(c0)) and torch.equal(s0, torch.zeros_like(s0))
    # cos/sin repeat across the two halves (emb = cat(freqs, freqs))
    assert torch.equal(cos[:, :64], cos[:, 64:]) and torch.equal(sin[:, :64], sin[:, 64:])


# --------------------------------------------------------------------------
# K logits (abx_rope_batched.py:189-202 with per-KV-head B_k, abx_rope_batched.py:81)
# --------------------------------------------------------------------------

def _complex_logits(q, x, inv_freq, positions):
    """Independent formulation: pair (i, i+64) as one complex number; the
    rotate_half RoPE at angle phi multiplies it by exp(i phi); a real dot of
    two such vectors is Re(sum conj(A) B).  q: [D] rotated query, x: [S, D]."""
    q = q.double()
    x = x.double()
    Q = torch.complex(q[:64], q[64:])
    X = torch.complex(x[:, :64], x[:, 64:])
    ang = positions.double()[:, None] * inv_freq.double()[None, :]     # exact-angle rotation
    Xr = X * torch.exp(1j * ang)
    return (Q.conj()[None, :] * Xr).real.sum(-1)


def test_k_logits_identity_basis_is_textbook_rope():
    g = torch.Generator().manual_seed(1)
    S = 37
    inv = o.rope_inv_freq()
    x = torch.randn(1, S, D, generator=g, dtype=torch.float64)
    q = torch.randn(1, 1, D, generator=g, dtype=torch.float64)
    cos, sin = o.rope_cos_sin(inv, torch.arange(S))
    lg = o.k_logits(q, [torch.eye(D, dtype=torch.float64)], [x], cos.double(), sin.double())
    ref = _complex_logits(q[0, 0], x[0], inv, torch.arange(S))
    # the oracle rotates with fp32 angles (as HF does); the complex form uses exact ones
    torch.testing.assert_close(lg[0, 0], ref, atol=1e-4 * ref.abs().max().item(), rtol=0)


def test_k_logits_bruteforce_tiny():
    g = torch.Generator().manual_seed(2)
    inv = o.rope_inv_freq()
    for S, ranks, Hq in [(1, [1], 1), (2, [3, 2], 2), (3, [4, 1], 4)]:
        Hkv = len(ranks)
        gs = Hq // Hkv
        q = torch.randn(1, Hq, D, generator=g, dtype=torch.float64)
        bk = [torch.randn(r, D, generator=g, dtype=torch.float64) for r in ranks]
        xk = [torch.randn(1, S, r, generator=g, dtype=torch.float64) for r in ranks]
        cos, sin = o.rope_cos_sin(inv, torch.arange(S))
        lg = o.k_logits(q, bk, xk, cos.double(), sin.double(), scale=0.5)
        for qh in range(Hq):
            h = qh // gs
            for s in range(S):
                k = [sum(float(xk[h][0, s, j]) * float(bk[h][j, d]) for j in range(ranks[h])) for d in range(D)]
                acc = 0.0
                for d in range(D):
                    c, sn = float(cos[s, d]), float(sin[s, d])
                    rh = -k[d + 64] if d < 64 else k[d - 64]
                    acc += float(q[0, qh, d]) * (k[d] * c + rh * sn)
                assert abs(float(lg[0, qh, s]) - 0.5 * acc) <= 1e-9 * (1 + abs(acc))


def test_k_logits_ragged_equals_zero_padded():
    g = torch.Generator().manual_seed(3)
    ranks = [5, 32, 17, 64]
    S = 50
    q = torch.randn(2, 4, D, generator=g, dtype=torch.float64)
    bk = [torch.randn(r, D, generator=g, dtype=torch.float64) for r in ranks]
    xk = [torch.randn(2, S, r, generator=g, dtype=torch.float64) for r in ranks]
    cos, sin = o.rope_cos_sin(o.rope_inv_freq(), torch.arange(S))
    a = o.k_logits(q, bk, xk, cos.double(), sin.double())
    R = 64
    bkp = [torch.cat([b, torch.zeros(R - b.shape[0], D, dtype=b.dtype)]) for b in bk]
    xkp = [torch.cat([x, torch.zeros(2, S, R - x.shape[2], dtype=x.dtype)], dim=2) for x in xk]
    b = o.k_logits(q, bkp, xkp, cos.double(), sin.double())
    assert torch.equal(a, b)


def test_k_logits_gqa_reads_kv_head_q_div_gs():
    g = torch.Generator().manual_seed(4)
    Hkv, gs, S, r = 2, 3, 9, 6
    q = torch.randn(1, Hkv * gs, D, generator=g, dtype=torch.float64)
    bk = [torch.randn(r, D, generator=g, dtype=torch.float64) for _ in range(Hkv)]
    xk = [torch.randn(1, S, r, generator=g, dtype=torch.float64) for _ in range(Hkv)]
    cos, sin = o.rope_cos_sin(o.rope_inv_freq(), torch.arange(S))
    full = o.k_logits(q, bk, xk, cos.double(), sin.double())
    for qh in range(Hkv * gs):
        one = o.k_logits(q[:, qh:qh + 1], [bk[qh // gs]], [xk[qh // gs]], cos.double(), sin.double())
        assert torch.equal(full[:, qh], one[:, 0])


# --------------------------------------------------------------------------
# full decode core vs SDPA on materialised K and V (the reorder identity,
# LlamaLoRaAttention_headwise.py:16, 126-142; model.py:458-487)
# --------------------------------------------------------------------------

def _sdpa_reference(q, bk, xk, xv, uv, cos, sin, mask=None):
    B, Hq, _ = q.shape
    Hkv = len(bk)
    gs = Hq // Hkv
    Rv = xv.shape[-1]
    U = uv.view(Hkv, D, Rv)
    outs = []
    for qh in range(Hq):
        h = qh // gs
        K = o.apply_rope(xk[h] @ bk[h], cos, sin)              # [B, S, D]
        V = xv @ U[h].transpose(0, 1)                           # [B, S, D]
        am = None if mask is None else mask[:, qh:qh + 1, None, :]
        outs.append(torch.nn.functional.scaled_dot_product_attention(
            q[:, qh:qh + 1, None, :], K[:, None], V[:, None], attn_mask=am)[:, 0, 0])
    return torch.stack(outs, dim=1)


@pytest.mark.parametrize("with_mask", [False, True])
def test_decode_attention_matches_sdpa(with_mask):
    g = torch.Generator().manual_seed(5)
    B, Hkv, gs, S, Rv = 2, 2, 2, 23, 40
    ranks = [7, 12]
    q = torch.randn(B, Hkv * gs, D, generator=g, dtype=torch.float64)
    bk = [torch.randn(r, D, generator=g, dtype=torch.float64) / math.sqrt(r) for r in ranks]
    xk = [torch.randn(B, S, r, generator=g, dtype=torch.float64) for r in ranks]
    xv = torch.randn(B, S, Rv, generator=g, dtype=torch.float64)
    uv = torch.randn(Hkv * D, Rv, generator=g, dtype=torch.float64) / math.sqrt(Rv)
    cos, sin = [t.double() for t in o.rope_cos_sin(o.rope_inv_freq(), torch.arange(S))]
    mask = None
    if with_mask:
        mask = torch.zeros(B, Hkv * gs, S, dtype=torch.float64)
        mask[:, :, ::3] = -1e9
    out, p, _ = o.decode_attention(q, bk, xk, xv, uv, cos, sin, mask=mask)
    ref = _sdpa_reference(q, bk, xk, xv, uv, cos, sin, mask)
    torch.testing.assert_close(out, ref, atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(p.sum(-1), torch.ones(B, Hkv * gs, dtype=torch.float64))


# --------------------------------------------------------------------------
# prefill (model.py:429-449 under a causal mask)
# --------------------------------------------------------------------------

def _prefill_case(seed, B=2, Hkv=2, gs=2, S=29, Rv=24, ranks=(8, 16)):
    g = torch.Generator().manual_seed(seed)
    bk = [torch.randn(r, D, generator=g, dtype=torch.float64) / math.sqrt(r) for r in ranks]
    xk = [torch.randn(B, S, r, generator=g, dtype=torch.float64) for r in ranks]
    xv = torch.randn(B, S, Rv, generator=g, dtype=torch.float64)
    uv = torch.randn(Hkv * D, Rv, generator=g, dtype=torch.float64) / math.sqrt(Rv)
    q = torch.randn(B, Hkv * gs, S, D, generator=g, dtype=torch.float64)
    cos, sin = [t.double() for t in o.rope_cos_sin(o.rope_inv_freq(), torch.arange(S))]
    return q, bk, xk, xv, uv, cos, sin


def test_prefill_matches_causal_sdpa():
    """pos0 = 0: torch SDPA with is_causal=True on K / V materialised per
    query head by the decode pin's own route."""
    q, bk, xk, xv, uv, cos, sin = _prefill_case(11)
    B, Hq, S, _ = q.shape
    gs = Hq // len(bk)
    U = uv.view(len(bk), D, -1)
    ref = torch.stack([torch.nn.functional.scaled_dot_product_attention(
        q[:, qh], o.apply_rope(xk[qh // gs] @ bk[qh // gs], cos, sin), xv @ U[qh // gs].t(), is_causal=True)
        for qh in range(Hq)], dim=1)
    out = o.prefill_attention(q, bk, xk, xv, uv, cos, sin)
    torch.testing.assert_close(out, ref, atol=1e-10, rtol=1e-10)


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float16])
def test_prefill_with_act_dtype_kv_matches_sdpa_on_rounded_kv(kv_dtype):
    """kv_dtype: K and V materialised per query head by the decode pin's route,
    rounded to the act dtype, then causal SDPA in fp64 -- and different from
    the unrounded result by about the rounding (it does round)."""
    q, bk, xk, xv, uv, cos, sin = _prefill_case(13)
    B, Hq, S, _ = q.shape
    gs = Hq // len(bk)
    U = uv.view(len(bk), D, -1)
    rnd = lambda t: t.to(kv_dtype).double()
    ref = torch.stack([torch.nn.functional.scaled_dot_product_attention(
        q[:, qh], rnd(o.apply_rope(xk[qh // gs] @ bk[qh // gs], cos, sin)), rnd(xv @ U[qh // gs].t()),
        is_causal=True) for qh in range(Hq)], dim=1)
    out = o.prefill_attention(q, bk, xk, xv, uv, cos, sin, kv_dtype=kv_dtype)
    torch.testing.assert_close(out, ref, atol=1e-10, rtol=1e-10)
    exact = o.prefill_attention(q, bk, xk, xv, uv, cos, sin)
    rel = float((out - exact).abs().mean() / exact.abs().mean())
    unit = 2.0 ** -9 if kv_dtype == torch.bfloat16 else 2.0 ** -12
    assert unit / 50 < rel < unit * 4, rel


def test_prefill_chunk_and_last_query_agree_with_full_and_decode():
    """Queries at positions pos0.. see what they see in a full prefill
    (chunked prefill), and the last query's row is the decode step."""
    q, bk, xk, xv, uv, cos, sin = _prefill_case(12)
    S = q.shape[2]
    full = o.prefill_attention(q, bk, xk, xv, uv, cos, sin)
    for pos0 in (1, 13, S - 1):
        part = o.prefill_attention(q[:, :, pos0:], bk, xk, xv, uv, cos, sin, pos0=pos0)
        torch.testing.assert_close(part, full[:, :, pos0:], atol=1e-12, rtol=1e-12)
    dec, _, _ = o.decode_attention(q[:, :, -1], bk, xk, xv, uv, cos, sin)
    torch.testing.assert_close(full[:, :, -1], dec, atol=1e-12, rtol=1e-12)


# --------------------------------------------------------------------------
# planted mistakes: each pin above must catch a plausible oracle bug
# --------------------------------------------------------------------------

def test_planted_causal_off_by_one_is_caught(monkeypatch):
    monkeypatch.setattr(o, "causal_visible",
                        lambda T, S, pos0: torch.arange(S)[None, :] < (pos0 + torch.arange(T))[:, None])
    with pytest.raises(AssertionError):
        test_prefill_matches_causal_sdpa()


def test_planted_value_head_layout_is_caught(monkeypatch):
    real = o.reconstruct_kv

    def wrong(bk, xk, xv, uv, cos, sin, dtype=torch.float64):
        K, V = real(bk, xk, xv, uv, cos, sin, dtype)
        B, H, S, _ = V.shape
        return K, V.transpose(1, 2).reshape(B, H, S, D)      # (S, H) order read as (H, S)
    monkeypatch.setattr(o, "reconstruct_kv", wrong)
    with pytest.raises(AssertionError):
        test_prefill_matches_causal_sdpa()

def test_planted_rotate_half_sign_is_caught(monkeypatch):
    monkeypatch.setattr(o, "rotate_half", lambda x: torch.cat((x[..., 64:], -x[..., :64]), dim=-1))
    with pytest.raises(AssertionError):
        test_k_logits_identity_basis_is_textbook_rope()


def test_planted_gqa_mapping_is_caught(monkeypatch):
    real = o.k_logits

    def wrong(q, bk, xk, cos, sin, scale=1.0, dtype=torch.float64):
        # query head q reads KV head q % Hkv (interleaved) instead of q // gs
        Hq, Hkv = q.shape[1], len(bk)
        gs = Hq // Hkv
        perm = [(qh % Hkv) * gs + qh // Hkv for qh in range(Hq)] if Hkv > 1 and gs > 1 else list(range(Hq))
        return real(q[:, perm], bk, xk, cos, sin, scale, dtype)[:, perm]
    monkeypatch.setattr(o, "k_logits", wrong)
    with pytest.raises(AssertionError):
        test_decode_attention_matches_sdpa(False)


def test_planted_nibble_order_is_caught(monkeypatch):
    def swapped(packed, r):
        p = packed.astype(np.int16)
        out = np.stack([((p >> 4) & 0xF) - 8, (p & 0xF) - 8], axis=-1).reshape(*packed.shape[:-1], -1)
        return out[..., :r].astype(np.int8)
    monkeypatch.setattr(o, "unpack_int4_ref", swapped)
    with pytest.raises(AssertionError):
        test_int4_ref_known_answers()


# --------------------------------------------------------------------------
# quantised-cache formats (bx_quant.py:75-86; build-defined int8 / int4-g64)
# --------------------------------------------------------------------------

def test_int4_ref_known_answers():
    # rank 2k lives in the low nibble of byte k, rank 2k+1 in the high nibble; value = nibble - 8
    packed = np.array([[0x00, 0xFF, 0x8F, 0x1A]], dtype=np.uint8)
    np.testing.assert_array_equal(o.unpack_int4_ref(packed, 8), [[-8, -8, 7, 7, 7, 0, 2, -7]])
    np.testing.assert_array_equal(o.unpack_int4_ref(packed, 5), [[-8, -8, 7, 7, 7]])


def test_int4_ref_exhaustive_table_and_round_trip():
    b = np.arange(256, dtype=np.uint8)[None, :]
    u = o.unpack_int4_ref(b, 512).reshape(256, 2)
    lo, hi = np.divmod(np.arange(256), 16)[1] - 8, np.divmod(np.arange(256), 16)[0] - 8
    np.testing.assert_array_equal(u[:, 0], lo)
    np.testing.assert_array_equal(u[:, 1], hi)
    np.testing.assert_array_equal(o.pack_int4_ref(u.reshape(1, 512)), b)
    rng = np.random.default_rng(0)
    v = rng.integers(-8, 8, size=(3, 7, 33)).astype(np.int8)     # odd rank: padded nibble
    np.testing.assert_array_equal(o.unpack_int4_ref(o.pack_int4_ref(v), 33), v)


def test_int4_ref_dequant_rounds_like_torch_fp16_multiply():
    rng = np.random.default_rng(1)
    n = np.tile(np.arange(-8, 8, dtype=np.int8), 64)[None, :]                 # [1, 1024]
    s = rng.uniform(1e-4, 4.0, size=(1, 1)).astype(np.float16)
    for _ in range(50):
        s = rng.uniform(1e-4, 4.0, size=(1, 1)).astype(np.float16)
        got = o.dequant_int4_ref(o.pack_int4_ref(n), s, n.shape[-1])
        want = (torch.from_numpy(n.astype(np.float32)).half() * torch.from_numpy(s)).numpy()
        np.testing.assert_array_equal(got, want)


def test_int8_sym_dequant_exact_and_quantiser_invariants():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((4, 9, 96)) * rng.uniform(0.01, 50, size=(4, 9, 1))).astype(np.float32)
    q, s = o.quant_int8_sym(x)
    assert q.dtype == np.int8 and q.min() >= -127 and q.max() <= 127
    assert s.shape == (4, 9, 1) and s.dtype == np.float16
    deq = o.dequant_int8_sym(q, s).astype(np.float64)
    want = (torch.from_numpy(q.astype(np.float32)).half() * torch.from_numpy(s)).numpy().astype(np.float64)
    np.testing.assert_array_equal(deq, want)
    # round to nearest: error <= s/2, plus the fp16 rounding of the dequantised value
    err = np.abs(deq - x)
    bound = s.astype(np.float64) / 2 * (1 + 1e-3) + np.abs(deq) * 2.0 ** -11
    assert (err <= bound).all()
    # idempotent: quantising the dequantised values with the same scale returns q
    q2 = np.clip(np.rint(deq / s.astype(np.float64)), -127, 127).astype(np.int8)
    np.testing.assert_array_equal(q2, q)


def test_int4_ref_quantiser_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 64)).astype(np.float32) * 3
    packed, s = o.quant_int4_ref(x)
    n = o.unpack_int4_ref(packed, 64)
    assert n.min() >= -8 and n.max() <= 7
    deq = o.dequant_int4_ref(packed, s, 64).astype(np.float64)
    bound = s.astype(np.float64) / 2 * (1 + 1e-3) + np.abs(deq) * 2.0 ** -11
    assert (np.abs(deq - x) <= bound).all()


@pytest.mark.parametrize("R", [64, 100, 1640])
def test_int4_g64_quantiser_invariants(R):
    rng = np.random.default_rng(R)
    x = rng.standard_normal((3, 5, R)).astype(np.float32)
    x[..., ::37] *= 10.0                                                     # outlier channels
    n, sc, zr = o.quant_int4_asym(x, 64)
    G = (R + 63) // 64
    assert sc.shape == (3, 5, G) and zr.shape == (3, 5, G)
    assert n.min() >= 0 and n.max() <= 15
    deq = o.dequant_int4_asym(n, sc, zr, 64).astype(np.float64)
    gidx = np.arange(R) // 64
    s = sc.astype(np.float64)[..., gidx]
    z = zr.astype(np.float64)[..., gidx]
    np.testing.assert_array_equal(deq, (n * s + z).astype(np.float16).astype(np.float64))
    # zero = fp16(min) may sit up to half an fp16 ulp above the true minimum
    bound = s / 2 * (1 + 1e-3) + np.abs(z) * 2.0 ** -11 + np.abs(deq) * 2.0 ** -11
    assert (np.abs(deq - x) <= bound).all()
