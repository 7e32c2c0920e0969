"""Write RoPE golden vectors with the installed third-party transformers
(5.15.0): the reference takes its RoPE from HF ``LlamaRotaryEmbedding``
(abx_rope_batched.py:18, 196-199; LlamaLoRaAttention_headwise.py:2-5) and its
``rotate_half`` (HF:models/llama/modeling_llama.py:130-134).

Outputs tests/golden/rope_fixtures.npz with, for the default config
(theta=1e4) and the llama3 config used by the Llama-3.1-8B-shaped workload
(theta=5e5, factor 8, low 1, high 4, original context 8192):
inv_freq [64], cos/sin [P, 128] fp32 at a fixed set of positions, and one
apply_rotary_pos_emb result on a seeded vector.

Run:  python tests/golden/make_rope_fixtures.py
"""
import os

import numpy as np
import torch
from transformers import LlamaConfig
from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb

POS = np.array([0, 1, 2, 3, 31, 32, 63, 64, 1000, 1023, 4095, 8191, 8192, 32767, 65535, 131071], dtype=np.int64)


def one(cfg, tag, out):
    rot = LlamaRotaryEmbedding(config=cfg)
    pos = torch.from_numpy(POS)[None, :]
    x = torch.zeros(1, 1, len(POS), 128, dtype=torch.float32)
    cos, sin = rot(x, pos)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 1, len(POS), 128, generator=g)
    k = torch.randn(1, 1, len(POS), 128, generator=g)
    qr, kr = apply_rotary_pos_emb(q, k, cos, sin)
    out[f"{tag}_inv_freq"] = rot.inv_freq.numpy().astype(np.float32)
    out[f"{tag}_attention_scaling"] = np.array(rot.attention_scaling, dtype=np.float64)
    out[f"{tag}_cos"] = cos[0].numpy()
    out[f"{tag}_sin"] = sin[0].numpy()
    out[f"{tag}_q"] = q[0, 0].numpy()
    out[f"{tag}_qrot"] = qr[0, 0].numpy()


def main():
    out = {"positions": POS}
    one(LlamaConfig(), "default", out)
    cfg3 = LlamaConfig(rope_theta=500000.0, max_position_embeddings=131072,
                       rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                     "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    one(cfg3, "llama3", out)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rope_fixtures.npz")
    np.savez(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
