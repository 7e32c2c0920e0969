"""Host-side logic of the Python layer that needs no GPU: the workspace
policy that keeps captured graphs valid, and the argument checks that must
raise before any kernel launch."""
import pytest
import torch

from starkv import ops
from starkv._lib import FMT_DENSE, StarKVError


def test_outgrown_workspace_is_retired_not_freed(monkeypatch):
    monkeypatch.setattr(ops, "_WS", {})
    monkeypatch.setattr(ops, "_WS_RETIRED", [])
    a = ops._workspace("cpu", 1000)
    assert a.numel() >= 1 << 20                       # minimum size
    assert ops._workspace("cpu", 5000).data_ptr() == a.data_ptr()   # reused while it fits
    b = ops._workspace("cpu", 3 << 20)
    assert b.data_ptr() != a.data_ptr() and b.numel() >= 3 << 20
    # the old buffer is kept alive: a graph captured with it keeps valid memory
    assert len(ops._WS_RETIRED) == 1 and ops._WS_RETIRED[0].data_ptr() == a.data_ptr()
    c = ops._workspace("cpu", b.numel() + 1)
    assert c.numel() >= 2 * b.numel()                 # geometric growth bounds the retired total
    assert [t.data_ptr() for t in ops._WS_RETIRED] == [a.data_ptr(), b.data_ptr()]


def _kspec(B=2, ranks=(16, 32), S=8):
    tot = S * sum(ranks)
    data = torch.zeros(B, tot, dtype=torch.float16)
    offs = [S * sum(ranks[:h]) for h in range(len(ranks))]
    bk = torch.zeros(len(ranks), max(ranks), 128, dtype=torch.float16)
    return ops.KLatentSpec(data, list(ranks), offs, list(ranks), tot, bk, [h * bk.stride(0) for h in range(len(ranks))],
                           128, fmt=FMT_DENSE)


@pytest.mark.parametrize("shape,msg", [
    ((2, 1, 1, 32), "heads"),           # fewer heads than the cache
    ((2, 2, 1, 16), "ranks"),           # rows shorter than the largest rank
    ((3, 2, 1, 32), "batch"),           # more sequences than the cache holds
])
def test_k_append_rejects_short_sources_before_launch(shape, msg):
    with pytest.raises(StarKVError, match=msg):
        ops.k_append(torch.zeros(*shape, dtype=torch.float16), _kspec(), 0, 8)


def test_v_append_rejects_short_sources_before_launch():
    v = ops.VLatentSpec.dense(torch.zeros(2, 8, 64, dtype=torch.float16))
    with pytest.raises(StarKVError, match="ranks"):
        ops.v_append(torch.zeros(2, 1, 48, dtype=torch.float16), v, 0, 8)
    with pytest.raises(StarKVError, match="batch"):
        ops.v_append(torch.zeros(4, 1, 64, dtype=torch.float16), v, 0, 8)


def test_device_position_tensors_are_checked():
    with pytest.raises(StarKVError, match="int32"):
        ops._pos_ptr(torch.zeros(1, dtype=torch.int64))
    with pytest.raises(StarKVError, match="int32"):
        ops._flag_ptr(torch.zeros(1, dtype=torch.int32))          # not a device tensor
    assert ops._flag_ptr(None) is None


@pytest.mark.parametrize("shape,ok", [
    ((4, 1, 1, 100), True), ((1, 1, 1, 100), True), ((4, 8, 1, 100), True),
    ((3, 1, 1, 100), False), ((4, 5, 1, 100), False), ((4, 1, 1, 90), False),
])
def test_mask_must_broadcast_to_batch_and_heads(shape, ok):
    m = torch.zeros(*shape)
    if ok:
        mm, _, sb, sh = ops._mask_args(m, B=4, S=100, Hq=8)
        assert mm.dim() == 3
        assert (sb == 0) == (shape[0] == 1) and (sh == 0) == (shape[1] == 1)
    else:
        with pytest.raises(StarKVError):
            ops._mask_args(m, B=4, S=100, Hq=8)
