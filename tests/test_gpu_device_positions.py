"""Run-time (device) positions that fall outside the cache or RoPE table.

Graph-replayed decode reads the write position from a device int, so the host
cannot reject an overrun before the launch.  The kernels then skip the rows
and set the caller's error flag; these tests force the condition from the
host (the device int is simply set past the capacity) and check that nothing
was written and that the flag was raised -- every kernel exits normally."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _flag():
    return torch.zeros(1, dtype=torch.int32, device="cuda")


def test_rope_apply_past_the_table_leaves_rows_and_sets_the_flag():
    from starkv import RopeConfig, rope_apply
    from starkv.rope import rope_table
    _, cap = rope_table(RopeConfig(), 64, "cuda")       # the table's own capacity bounds the positions
    x = torch.randn(2, 4, 1, 128, device="cuda").half()
    before = x.clone()
    flag = _flag()
    pos = torch.tensor([cap], dtype=torch.int32, device="cuda")
    rope_apply(x, RopeConfig(), pos0_device=pos, max_positions=64, error_flag=flag)
    torch.cuda.synchronize()
    assert torch.equal(x, before)
    assert int(flag.item()) == 1
    # an in-range position rotates and leaves the flag alone
    flag.zero_()
    pos.fill_(cap - 1)
    rope_apply(x, RopeConfig(), pos0_device=pos, max_positions=64, error_flag=flag)
    torch.cuda.synchronize()
    assert not torch.equal(x, before)
    assert int(flag.item()) == 0


@pytest.mark.parametrize("fmt", ["dense", "int8_g64", "reference"])
def test_cache_writers_past_capacity_write_nothing_and_set_the_flag(fmt):
    from starkv.cache import LatentCache
    B, ranks, Rv, cap = 2, [32, 16, 48], 256, 40
    cache = LatentCache(B, ranks, Rv, cap, torch.float16, "cuda", fmt=fmt)
    bk = torch.randn(len(ranks), max(ranks), 128, device="cuda").half()
    k_new = torch.randn(B, 1, sum(ranks), device="cuda").half()
    v_new = torch.randn(B, 1, Rv, device="cuda").half()
    snap = [t.clone() for t in (cache.k_data, cache.v_data)]
    flag = _flag()
    pos = torch.tensor([cap], dtype=torch.int32, device="cuda")
    cache.append_at(k_new, v_new, bk, pos, error_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    assert torch.equal(cache.k_data, snap[0]) and torch.equal(cache.v_data, snap[1])
    flag.zero_()
    pos.fill_(cap - 1)
    cache.append_at(k_new, v_new, bk, pos, error_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    assert not torch.equal(cache.v_data, snap[1])
