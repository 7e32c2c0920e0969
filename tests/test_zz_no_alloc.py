"""The allocation-free decode entry point (starkv_decode_attention_noalloc:
workspace in the library's own device array) against starkv_decode_attention
on the same inputs: identical outputs (the same kernels, deterministic), and
both within the oracle's gates.  Two calls in a row, the second smaller, so
the shared array's leftovers from the first call cannot leak into the second."""
import pytest
import torch

from _util import cfg2_ranks, check_output, make_case, oracle_decode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_noalloc_decode_matches_the_workspace_entry_point(dtype):
    from starkv import RopeConfig, decode_attention
    from starkv._lib import NOALLOC_SCRATCH_BYTES, lib
    rope = RopeConfig()
    cases = [make_case(4, 32, 32, 3000, cfg2_ranks(), 1640, dtype=dtype, seed=31),      # first call: larger
             make_case(2, 32, 8, 700, [32, 128, 32, 80, 32, 64, 80, 64], 512, dtype=dtype, seed=32)]
    assert NOALLOC_SCRATCH_BYTES == 128 << 20
    for i, case in enumerate(cases):
        print(f"[noalloc] call {i}: B={case.B} Hq={case.Hq} Hkv={case.Hkv} S={case.S} Rv={case.Rv} {dtype}", flush=True)
        out = torch.full((case.B, case.Hq, 128), float("nan"), dtype=dtype, device="cuda")   # every element written
        got = decode_attention(case.q, case.kspec, case.xv, case.uv, rope=rope, out=out, noalloc=True)
        want = decode_attention(case.q, case.kspec, case.xv, case.uv, rope=rope)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert torch.equal(got, want)
        ref, _, _ = oracle_decode(case, rope=rope)
        check_output(got, ref)
