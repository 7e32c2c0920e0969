"""starkv: MI355X (gfx950) decode and prefill attention over STAR-KV low-rank latent caches.

The compute lives in libstarkv.so (HIP kernels behind the C ABI of
include/starkv.h); this package binds it to torch tensors.
"""
from ._lib import StarKVError, lib
from .ops import KLatentSpec, VLatentSpec, decode_attention, k_logits, prefill_attention, pv_latent, rope_apply
from .rope import RopeConfig, rope_table

__all__ = ["StarKVError", "lib", "KLatentSpec", "VLatentSpec", "decode_attention", "k_logits", "prefill_attention",
           "pv_latent", "rope_apply",
           "RopeConfig", "rope_table"]
