"""C-ABI checks of libstarkv.so that need no GPU.

The library must load, export every function include/starkv.h declares, agree
with the ctypes mirrors on struct layout, and reject bad arguments with the
documented status codes.  Validation runs before any HIP call, so every call
below returns before touching a device (device pointers are never
dereferenced on the host; fake addresses are enough).
"""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

from starkv import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "starkv.h")

OK, ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_ALIGN, ERR_RANK, ERR_WORKSPACE, ERR_LIMIT, ERR_FORMAT = 0, -1, -2, -3, -4, -5, -6, -7, -8
FAKE = 0x7F0000000000          # 256-byte aligned stand-in for a device address


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(starkv_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_function():
    lib = L.lib()
    decl = declared_functions()
    assert len(decl) >= 11
    missing = [n for n in decl if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(L.EXPORTS) == decl


def test_version_and_status_strings():
    lib = L.lib()
    m = re.search(r"#define\s+STARKV_ABI_VERSION\s+(\d+)", open(HEADER).read())
    header_version = int(m.group(1))
    # the library, the header and the ctypes mirrors must agree: a struct
    # layout change bumps all three together
    assert lib.starkv_abi_version() == header_version == L.ABI_VERSION == 5
    for code in (OK, ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_ALIGN, ERR_RANK, ERR_WORKSPACE, ERR_LIMIT, ERR_FORMAT):
        s = lib.starkv_status_string(code).decode()
        assert s and s != "unknown error"
    assert lib.starkv_status_string(-99).decode() == "unknown error"


_C_LAYOUT = r"""
#include <stdio.h>
#include <stddef.h>
#include "starkv.h"
#define F(T, f) printf(#T " " #f " %zu\n", offsetof(T, f));
#define S(T) printf(#T " sizeof %zu\n", sizeof(T));
int main(void) {
  S(starkv_klatent) F(starkv_klatent, rank) F(starkv_klatent, data) F(starkv_klatent, scale_stride_h) F(starkv_klatent, bk_row_stride)
  F(starkv_klatent, split) F(starkv_klatent, data2) F(starkv_klatent, pos_stride2) F(starkv_klatent, scale2_stride_h)
  S(starkv_klogits_desc) F(starkv_klogits_desc, q) F(starkv_klogits_desc, k) F(starkv_klogits_desc, rope_table)
  F(starkv_klogits_desc, scale) F(starkv_klogits_desc, mask) F(starkv_klogits_desc, out) F(starkv_klogits_desc, out_stride_h)
  S(starkv_vlatent) F(starkv_vlatent, data) F(starkv_vlatent, split) F(starkv_vlatent, data2) F(starkv_vlatent, zero) F(starkv_vlatent, capacity)
  S(starkv_pv_desc) F(starkv_pv_desc, p) F(starkv_pv_desc, v) F(starkv_pv_desc, out_stride_h)
  S(starkv_decode_desc) F(starkv_decode_desc, k) F(starkv_decode_desc, v) F(starkv_decode_desc, uv)
  F(starkv_decode_desc, rope_table) F(starkv_decode_desc, scale) F(starkv_decode_desc, mask) F(starkv_decode_desc, out_dtype)
  F(starkv_decode_desc, out_stride_h) F(starkv_decode_desc, last_pos_device)
  S(starkv_k_append_desc) F(starkv_k_append_desc, k) F(starkv_k_append_desc, src_head_offset)
  F(starkv_k_append_desc, pos0_device) F(starkv_k_append_desc, error_flag)
  S(starkv_v_append_desc) F(starkv_v_append_desc, v) F(starkv_v_append_desc, pos0_device)
  F(starkv_v_append_desc, error_flag)
  S(starkv_rope_apply_desc) F(starkv_rope_apply_desc, x) F(starkv_rope_apply_desc, rope_table)
  F(starkv_rope_apply_desc, pos0) F(starkv_rope_apply_desc, pos0_device) F(starkv_rope_apply_desc, error_flag)
  S(starkv_prefill_desc) F(starkv_prefill_desc, pos0) F(starkv_prefill_desc, dtype) F(starkv_prefill_desc, q)
  F(starkv_prefill_desc, q_stride_t) F(starkv_prefill_desc, k) F(starkv_prefill_desc, v) F(starkv_prefill_desc, uv)
  F(starkv_prefill_desc, rope_table) F(starkv_prefill_desc, scale) F(starkv_prefill_desc, out)
  F(starkv_prefill_desc, out_stride_t)
  S(starkv_rms_norm_desc) F(starkv_rms_norm_desc, x) F(starkv_rms_norm_desc, residual_out_stride)
  F(starkv_rms_norm_desc, weight) F(starkv_rms_norm_desc, eps) F(starkv_rms_norm_desc, out_stride)
  S(starkv_silu_mul_desc) F(starkv_silu_mul_desc, gate) F(starkv_silu_mul_desc, up_stride) F(starkv_silu_mul_desc, out)
  S(starkv_skinny_gemm_desc) F(starkv_skinny_gemm_desc, epilogue) F(starkv_skinny_gemm_desc, x)
  F(starkv_skinny_gemm_desc, w_stride) F(starkv_skinny_gemm_desc, out_stride) F(starkv_skinny_gemm_desc, w_packed)
  F(starkv_skinny_gemm_desc, rms_eps)
  return 0;
}
"""

_PY = {"starkv_klatent": L.KLatent, "starkv_klogits_desc": L.KLogitsDesc, "starkv_vlatent": L.VLatent,
       "starkv_pv_desc": L.PVDesc, "starkv_decode_desc": L.DecodeDesc,
       "starkv_prefill_desc": L.PrefillDesc, "starkv_k_append_desc": L.KAppendDesc,
       "starkv_v_append_desc": L.VAppendDesc, "starkv_rope_apply_desc": L.RopeApplyDesc,
       "starkv_rms_norm_desc": L.RmsNormDesc, "starkv_silu_mul_desc": L.SiluMulDesc,
       "starkv_skinny_gemm_desc": L.SkinnyGemmDesc}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_ctypes_struct_layout_matches_the_c_compiler(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(_C_LAYOUT)
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    n = 0
    for line in filter(None, lines):
        cname, field, val = line.split()
        py = _PY[cname]
        got = ctypes.sizeof(py) if field == "sizeof" else getattr(py, field).offset
        assert got == int(val), (cname, field, got, val)
        n += 1
    assert n > 20


# ---------------------------------------------------------------- validation

def _klatent(ranks, keep):
    Hkv = len(ranks)
    keep += [L.int_array(ranks), L.i64_array([h * 4096 * 64 for h in range(Hkv)]),
             L.i64_array([64] * Hkv), L.i64_array([sum(ranks[:h]) * 128 for h in range(Hkv)])]
    return L.KLatent(n_kv_heads=Hkv, rank=keep[-4], head_offset=keep[-3], pos_stride=keep[-2],
                     stride_b=Hkv * 4096 * 64, format=L.FMT_DENSE, data=FAKE, scale=None,
                     scale_stride_b=0, scale_stride_h=0, bk=FAKE, bk_head_offset=keep[-1], bk_row_stride=128)


def _decode_desc(keep, B=2, Hq=8, Hkv=8, S=1000, Rv=256, ranks=None):
    ranks = ranks or [32] * Hkv
    d = L.DecodeDesc()
    d.batch, d.n_q_heads, d.head_dim, d.seq_len, d.dtype = B, Hq, 128, S, L.F16
    d.q, d.q_stride_b, d.q_stride_h = FAKE, Hq * 128, 128
    d.k = _klatent(ranks, keep)
    d.v = L.VLatent(rank=Rv, format=L.FMT_DENSE, data=FAKE, stride_b=S * Rv, stride_s=Rv)
    d.uv, d.uv_row_stride = FAKE, Rv
    d.rope_table, d.rope_max_positions = FAKE, 4096
    d.scale = 128 ** -0.5
    d.out, d.out_dtype, d.out_stride_b, d.out_stride_h = FAKE, 0, Hq * 128, 128
    return d


def _call(d, ws=None, nbytes=0):
    return L.lib().starkv_decode_attention(ctypes.byref(d), ws, nbytes, None)


def test_noalloc_decode_refuses_workspaces_beyond_its_array():
    """starkv_decode_attention_noalloc validates like the workspace entry point
    and refuses, before touching a device, any descriptor whose workspace
    would not fit its fixed device array."""
    lib = L.lib()
    assert lib.starkv_decode_attention_noalloc(None, None) == ERR_NULL
    keep = []
    d = _decode_desc(keep, B=32, Hq=32, Hkv=32, S=32768, Rv=1640)
    d.rope_max_positions = 1 << 16
    need = lib.starkv_decode_workspace_bytes(ctypes.byref(d))
    assert need > L.NOALLOC_SCRATCH_BYTES
    assert lib.starkv_decode_attention_noalloc(ctypes.byref(d), None) == ERR_LIMIT
    d.head_dim = 64
    assert lib.starkv_decode_attention_noalloc(ctypes.byref(d), None) == ERR_SHAPE
    m = re.search(r"#define\s+STARKV_NOALLOC_SCRATCH_BYTES\s+\((\d+)u << (\d+)\)", open(HEADER).read())
    assert int(m.group(1)) << int(m.group(2)) == L.NOALLOC_SCRATCH_BYTES


def test_valid_descriptor_sizes_a_workspace_and_asks_for_it():
    keep = []
    d = _decode_desc(keep)
    need = L.lib().starkv_decode_workspace_bytes(ctypes.byref(d))
    assert need > 0 and need % 256 == 0
    assert _call(d) == ERR_WORKSPACE
    assert _call(d, FAKE, need - 1) == ERR_WORKSPACE
    assert _call(d, FAKE + 16, need) == ERR_ALIGN


@pytest.mark.parametrize("field,value,code", [
    ("batch", 0, ERR_SHAPE),
    ("seq_len", 0, ERR_SHAPE),
    ("seq_len", 5000, ERR_SHAPE),          # beyond rope_max_positions
    ("head_dim", 64, ERR_SHAPE),
    ("dtype", L.F32, ERR_DTYPE),
    ("n_q_heads", 12, ERR_SHAPE),          # not a multiple of n_kv_heads
    ("n_q_heads", 72, ERR_LIMIT),          # up to 64 query heads (two P.V head groups)
    ("q", None, ERR_NULL),
    ("uv", None, ERR_NULL),
    ("out", None, ERR_NULL),
    ("rope_table", None, ERR_NULL),
    ("out_dtype", L.I8, ERR_DTYPE),
    ("uv_row_stride", 100, ERR_SHAPE),
    ("mask_dtype", L.I8, ERR_DTYPE),
])
def test_decode_rejects(field, value, code):
    keep = []
    d = _decode_desc(keep)
    setattr(d, field, value)
    if field == "mask_dtype":
        d.mask = FAKE
    assert _call(d) == code
    assert L.lib().starkv_decode_workspace_bytes(ctypes.byref(d)) == 0


@pytest.mark.parametrize("what,code", [
    ("rank0", ERR_RANK), ("rank129", ERR_RANK), ("format", ERR_FORMAT), ("pos_stride", ERR_SHAPE),
    ("k_null", ERR_NULL), ("int8_noscale", ERR_NULL), ("v_rank", ERR_RANK), ("v_format", ERR_FORMAT),
    ("v_stride", ERR_SHAPE), ("kv_heads", ERR_LIMIT),
])
def test_decode_rejects_latent_descriptions(what, code):
    keep = []
    d = _decode_desc(keep)
    if what == "rank0":
        d.k.rank[3] = 0
    elif what == "rank129":
        d.k.rank[0] = 129
    elif what == "format":
        d.k.format = 9
    elif what == "pos_stride":
        d.k.pos_stride[1] = 16
    elif what == "k_null":
        d.k.data = None
    elif what == "int8_noscale":
        d.k.format = L.FMT_INT8_SYM
    elif what == "v_rank":
        d.v.rank = 0
    elif what == "v_format":
        d.v.format = 7
    elif what == "v_stride":
        d.v.stride_s = 10
    elif what == "kv_heads":
        d = _decode_desc(keep, Hq=65 * 2, Hkv=65, ranks=[8] * 65)
    assert _call(d) == code


def test_rope_build_and_pv_validation():
    lib = L.lib()
    assert lib.starkv_rope_table_bytes(0) == 0
    assert lib.starkv_rope_table_bytes(1) == lib.starkv_rope_table_bytes(32) == 8192     # one 32-position tile
    assert lib.starkv_rope_table_bytes(33) == 2 * 8192
    inv = (ctypes.c_float * 64)(*([1.0] * 64))
    assert lib.starkv_rope_build(None, 1.0, 32, FAKE, 8192, None) == ERR_NULL
    assert lib.starkv_rope_build(inv, 1.0, 64, FAKE, 8192, None) == ERR_WORKSPACE
    assert lib.starkv_rope_build(inv, 1.0, 32, FAKE + 8, 8192, None) == ERR_ALIGN
    assert lib.starkv_rope_build(inv, 1.0, 0, FAKE, 8192, None) == ERR_SHAPE
    p = L.PVDesc(batch=2, n_heads=32, seq_len=100, dtype=L.F16, p=FAKE, p_stride_b=3200, p_stride_h=100,
                 v=L.VLatent(rank=256, format=L.FMT_DENSE, data=FAKE, stride_b=25600, stride_s=256),
                 out=FAKE, out_stride_b=8192, out_stride_h=256)
    need = lib.starkv_pv_latent_workspace_bytes(ctypes.byref(p))
    assert need > 0
    assert lib.starkv_pv_latent(ctypes.byref(p), None, 0, None) == ERR_WORKSPACE
    # 33..64 heads take two head groups: a larger workspace; more than 64 are refused
    p.n_heads = 40
    need40 = lib.starkv_pv_latent_workspace_bytes(ctypes.byref(p))
    assert need40 > need
    assert lib.starkv_pv_latent(ctypes.byref(p), FAKE, need, None) == ERR_WORKSPACE
    p.n_heads = 65
    assert lib.starkv_pv_latent(ctypes.byref(p), FAKE, need40, None) == ERR_LIMIT
    p.n_heads, p.p = 32, None
    assert lib.starkv_pv_latent(ctypes.byref(p), FAKE, need, None) == ERR_NULL
    # group-64 int4 rows are addressed with a 24-bit row multiply: pitches of
    # 16 MB or more are refused
    p.p = FAKE
    p.v = L.VLatent(rank=256, format=L.FMT_INT4_G64, data=FAKE, stride_b=1 << 30, stride_s=128, scale=FAKE,
                    scale_stride_b=1 << 20, scale_stride_s=4, zero=FAKE)
    need = lib.starkv_pv_latent_workspace_bytes(ctypes.byref(p))
    assert need > 0
    assert lib.starkv_pv_latent(ctypes.byref(p), None, 0, None) == ERR_WORKSPACE
    p.v.stride_s = 1 << 24
    assert lib.starkv_pv_latent(ctypes.byref(p), FAKE, need, None) == ERR_LIMIT
    p.v.stride_s, p.v.scale_stride_s = 128, 1 << 23
    assert lib.starkv_pv_latent(ctypes.byref(p), FAKE, need, None) == ERR_LIMIT


def test_k_logits_validation():
    lib = L.lib()
    keep = []
    d = L.KLogitsDesc(batch=1, n_q_heads=8, head_dim=128, seq_len=64, dtype=L.F16, q=FAKE,
                      q_stride_b=1024, q_stride_h=128, k=_klatent([16] * 8, keep), rope_table=FAKE,
                      rope_max_positions=64, scale=1.0, out=FAKE, out_dtype=L.F32, out_stride_b=512, out_stride_h=64)
    assert lib.starkv_k_logits_workspace_bytes(ctypes.byref(d)) == 0
    for field, value, code in [("out_dtype", L.I8, ERR_DTYPE), ("q", None, ERR_NULL), ("seq_len", 65, ERR_SHAPE),
                               ("n_q_heads", 7, ERR_SHAPE), ("head_dim", 96, ERR_SHAPE)]:
        old = getattr(d, field)
        setattr(d, field, value)
        assert lib.starkv_k_logits(ctypes.byref(d), None, 0, None) == code, field
        setattr(d, field, old)
    assert lib.starkv_k_logits(None, None, 0, None) == ERR_NULL


def test_k_logits_repack_workspace():
    """Dense K whose rows the streaming K-logit kernels cannot read (rank 102,
    the reference abx benchmark's: 204-byte rows) asks for a workspace that
    holds a padded copy ([B][Hkv][S][208 bytes]) and refuses to run without it;
    ranks that are multiples of 8 on aligned rows need none."""
    lib = L.lib()
    keep = []
    k = _klatent([102] * 8, keep)
    keep.append(L.i64_array([102] * 8))
    k.pos_stride = keep[-1]
    d = L.KLogitsDesc(batch=2, n_q_heads=32, head_dim=128, seq_len=64, dtype=L.F16, q=FAKE,
                      q_stride_b=32 * 128, q_stride_h=128, k=k, rope_table=FAKE, rope_max_positions=64,
                      scale=1.0, out=FAKE, out_dtype=L.F16, out_stride_b=32 * 64, out_stride_h=64)
    need = lib.starkv_k_logits_workspace_bytes(ctypes.byref(d))
    assert need >= 2 * 8 * 64 * 208
    assert lib.starkv_k_logits(ctypes.byref(d), None, 0, None) == ERR_WORKSPACE
    assert lib.starkv_k_logits(ctypes.byref(d), FAKE, need - 1, None) == ERR_WORKSPACE
    assert lib.starkv_k_logits(ctypes.byref(d), FAKE + 16, need, None) == ERR_ALIGN
    d.k = _klatent([104] * 8, keep)
    assert lib.starkv_k_logits_workspace_bytes(ctypes.byref(d)) == 0


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", os.path.join(ROOT, "no-such-dir", "libstarkv.so"))
    with pytest.raises(L.StarKVError, match="no fallback"):
        L.lib()


def test_dropins_refuse_cpu_tensors():
    import torch
    from starkv.abx_rope_batched import abx
    a = torch.zeros(1, 2, 1, 128, dtype=torch.float16)
    b = torch.zeros(2, 16, 128, dtype=torch.float16)
    x = torch.zeros(1, 2, 10, 16, dtype=torch.float16)
    with pytest.raises(L.StarKVError, match="no CPU path"):
        abx(a, b, x)
    with pytest.raises(L.StarKVError):
        abx(a[0], b, x)                      # wrong rank
    with pytest.raises(L.StarKVError):
        abx(a, b.float(), x)                 # mixed dtypes


def test_cache_writer_validation():
    lib = L.lib()
    keep = []
    d = L.KAppendDesc(batch=2, n_tokens=4, pos0=10, capacity=12, dtype=L.F16, src=FAKE,
                      src_stride_b=8 * 4 * 32, src_stride_h=4 * 32, src_stride_t=32, k=_klatent([32] * 8, keep))
    assert lib.starkv_k_append(ctypes.byref(d), None) == ERR_SHAPE          # 10 + 4 > 12
    d.capacity = 14
    d.dtype = L.F32
    assert lib.starkv_k_append(ctypes.byref(d), None) == ERR_DTYPE
    d.dtype, d.src = L.F16, None
    assert lib.starkv_k_append(ctypes.byref(d), None) == ERR_NULL
    d.src = FAKE
    d.k.format = L.FMT_INT8_SYM                                            # quantised without scales
    assert lib.starkv_k_append(ctypes.byref(d), None) == ERR_NULL
    v = L.VAppendDesc(batch=1, n_tokens=1, pos0=0, capacity=8, dtype=L.F16, src=FAKE, src_stride_b=64,
                      src_stride_t=64, v=L.VLatent(rank=64, format=L.FMT_INT4_G64, data=FAKE, stride_b=8 * 32,
                                                    stride_s=32, scale=FAKE, scale_stride_b=8, scale_stride_s=1))
    assert lib.starkv_v_append(ctypes.byref(v), None) == ERR_NULL           # group-64 without zero points
    v.v.zero, v.v.stride_s = FAKE, 30
    assert lib.starkv_v_append(ctypes.byref(v), None) == ERR_SHAPE          # row shorter than rank/2 bytes
    v.v.stride_s, v.v.scale = 32, FAKE + 1                                  # fp16 scales at an odd address
    assert lib.starkv_v_append(ctypes.byref(v), None) == ERR_ALIGN
    assert lib.starkv_v_append(None, None) == ERR_NULL
    # the combined writer reports each description's own status, and a dtype mismatch
    d.k.format = L.FMT_DENSE
    assert lib.starkv_decode_append(ctypes.byref(d), ctypes.byref(v), None, None) == ERR_ALIGN
    assert lib.starkv_decode_append(None, ctypes.byref(v), None, None) == ERR_NULL
    v.v.scale = FAKE
    q = L.RopeApplyDesc(batch=2, n_heads=8, n_tokens=4, dtype=L.BF16, x=FAKE, stride_b=8 * 4 * 128,
                        stride_h=4 * 128, stride_t=128, rope_table=FAKE, rope_max_positions=16, pos0=10)
    assert lib.starkv_decode_append(ctypes.byref(d), ctypes.byref(v), ctypes.byref(q), None) == ERR_DTYPE
    q.rope_max_positions = 12
    assert lib.starkv_decode_append(ctypes.byref(d), ctypes.byref(v), ctypes.byref(q), None) == ERR_SHAPE


# ---------------------------------------------------------------- prefill validation

def _prefill_desc(keep, B=2, Hq=8, Hkv=4, T=100, pos0=20, Rv=64, ranks=None):
    ranks = ranks or [32] * Hkv
    d = L.PrefillDesc()
    d.batch, d.n_q_heads, d.head_dim, d.n_tokens, d.pos0, d.dtype = B, Hq, 128, T, pos0, L.F16
    d.q, d.q_stride_b, d.q_stride_h, d.q_stride_t = FAKE, Hq * T * 128, T * 128, 128
    d.k = _klatent(ranks, keep)
    S = pos0 + T
    d.v = L.VLatent(rank=Rv, format=L.FMT_DENSE, data=FAKE, stride_b=S * Rv, stride_s=Rv)
    d.uv, d.uv_row_stride = FAKE, Rv
    d.rope_table, d.rope_max_positions = FAKE, 4096
    d.scale = 128 ** -0.5
    d.out, d.out_stride_b, d.out_stride_h, d.out_stride_t = FAKE, Hq * T * 128, T * 128, 128
    return d


def test_prefill_workspace_holds_the_reconstructed_k_and_v():
    keep = []
    d = _prefill_desc(keep)
    need = L.lib().starkv_prefill_workspace_bytes(ctypes.byref(d))
    assert need == 2 * 2 * 4 * 128 * 128 * 2          # B * Hkv * round_up(120, 64) * 128 fp16, twice
    call = lambda ws, n: L.lib().starkv_prefill_attention(ctypes.byref(d), ws, n, None)
    assert call(None, 0) == ERR_WORKSPACE
    assert call(FAKE, need - 1) == ERR_WORKSPACE
    assert call(FAKE + 16, need) == ERR_ALIGN


@pytest.mark.parametrize("what,code", [
    ("n_tokens0", ERR_SHAPE), ("pos0_neg", ERR_SHAPE), ("rope_short", ERR_SHAPE), ("head_dim", ERR_SHAPE),
    ("k_format", ERR_FORMAT), ("v_format", ERR_FORMAT), ("k_split_format", ERR_FORMAT),
    ("q_stride", ERR_ALIGN), ("q_null", ERR_NULL), ("gqa", ERR_SHAPE),
    ("dtype", ERR_DTYPE),
])
def test_prefill_rejects(what, code):
    keep = []
    d = _prefill_desc(keep)
    if what == "n_tokens0":
        d.n_tokens = 0
    elif what == "pos0_neg":
        d.pos0 = -1
    elif what == "rope_short":
        d.rope_max_positions = 119
    elif what == "head_dim":
        d.head_dim = 64
    elif what == "k_format":
        d.k.format, d.k.scale = 77, FAKE
    elif what == "v_format":
        d.v.format, d.v.scale = 77, FAKE
    elif what == "k_split_format":
        d.k.format, d.k.scale, d.k.split, d.k.split_format = L.FMT_INT4_REF, FAKE, 16, L.FMT_INT4_G64
    elif what == "q_stride":
        d.q_stride_t = 132
    elif what == "q_null":
        d.q = None
    elif what == "gqa":
        d.n_q_heads = 6
    elif what == "dtype":
        d.dtype = L.F32
    assert L.lib().starkv_prefill_attention(ctypes.byref(d), FAKE, 1 << 30, None) == code
    assert L.lib().starkv_prefill_workspace_bytes(ctypes.byref(d)) == 0


@pytest.mark.parametrize("what,extra", [
    # ranks or rows the reconstruction kernels cannot read in place are
    # repacked into aligned workspace rows after the reconstructed K and V:
    # (kind of copy, its bytes)
    ("k_rank_odd", 2 * 4 * 120 * 64),            # K: B x Hkv x S rows of 32 ranks (rank 20 padded) x 2 B
    ("k_offset_odd", 2 * 4 * 120 * 64),          # K: a head offset that is not a multiple of 8 elements
    ("v_rank_odd", 2 * 120 * 128 + 4 * 128 * 128),   # V rows of 64 ranks (60 padded) and U_v rows of 64
    ("uv_stride", 4 * 128 * 128),                # U_v rows 68 elements apart (not 16-byte rows)
    ("v_data_odd", 2 * 120 * 128),               # V data 2 bytes into its buffer
])
def test_prefill_repacks_what_it_cannot_read_in_place(what, extra):
    keep = []
    d = _prefill_desc(keep)
    base = L.lib().starkv_prefill_workspace_bytes(ctypes.byref(d))
    if what == "k_rank_odd":
        d.k.rank[2] = 20
    elif what == "k_offset_odd":
        d.k.head_offset[1] += 4
    elif what == "v_rank_odd":
        d.v.rank, d.uv_row_stride = 60, 60
    elif what == "uv_stride":
        d.uv_row_stride = 68
    elif what == "v_data_odd":
        d.v.data = FAKE + 2
    assert L.lib().starkv_prefill_workspace_bytes(ctypes.byref(d)) == base + extra


def test_quantised_layouts_take_any_rank_and_alignment():
    """The reference's bx check shape (bx_quant.py:224-248): rank 1228 over a
    256-rank upper block, 486-byte lower rows; odd K ranks; unaligned rows."""
    lib = L.lib()
    v = L.VLatent(rank=1228, format=L.FMT_INT4_REF, data=FAKE, stride_b=4096 * 128, stride_s=128,
                  scale=FAKE, scale_stride_b=4096, scale_stride_s=1, split=256, split_format=L.FMT_INT4_REF,
                  data2=FAKE + 2, stride2_b=4096 * 486, stride2_s=486, scale2=FAKE, scale2_stride_b=4096,
                  scale2_stride_s=1)
    d = L.PVDesc(batch=16, n_heads=32, seq_len=4096, dtype=L.F16, p=FAKE, p_stride_b=32 * 4096, p_stride_h=4096,
                 v=v, out=FAKE, out_stride_b=32 * 1228, out_stride_h=1228)
    assert lib.starkv_pv_latent_workspace_bytes(ctypes.byref(d)) > 0
    d.v.stride2_s = 485                                                     # shorter than ceil(972 / 2)
    assert lib.starkv_pv_latent(ctypes.byref(d), FAKE, 1 << 30, None) == ERR_SHAPE
    d.v.stride2_s, d.v.split = 486, 252                                     # split not a multiple of 8
    assert lib.starkv_pv_latent(ctypes.byref(d), FAKE, 1 << 30, None) == ERR_SHAPE
    keep = []
    dd = _decode_desc(keep, ranks=[37, 60, 5, 64, 17, 50, 33, 1])
    dd.k.format, dd.k.scale, dd.k.scale_stride_b, dd.k.scale_stride_h = L.FMT_INT8_SYM, FAKE, 8 * 1024, 1024
    dd.k.pos_stride[0] = 37
    dd.k.head_offset[0] = 3
    assert lib.starkv_decode_workspace_bytes(ctypes.byref(dd)) > 0
    dd.k.pos_stride[0] = 36                                                 # row shorter than its 37 ranks
    assert _call(dd) == ERR_SHAPE


def test_rope_apply_validation():
    lib = L.lib()
    d = L.RopeApplyDesc(batch=1, n_heads=2, n_tokens=10, dtype=L.F16, x=FAKE, stride_b=2560, stride_h=1280,
                        stride_t=128, rope_table=FAKE, rope_max_positions=64, pos0=60)
    assert lib.starkv_rope_apply(ctypes.byref(d), None) == ERR_SHAPE        # positions 60..69 past the table
    d.pos0 = 0
    d.x = None
    assert lib.starkv_rope_apply(ctypes.byref(d), None) == ERR_NULL
    d.x, d.dtype = FAKE, L.F32
    assert lib.starkv_rope_apply(ctypes.byref(d), None) == ERR_DTYPE
    # one thread per (row, frequency): grids of 2^32 threads or more are refused
    # before any launch (a device position lifts the host-side table check)
    d.dtype, d.pos0_device = L.F16, FAKE
    d.batch, d.n_heads, d.n_tokens = 1 << 16, 64, 1 << 10          # 2^32 * 64 / 64 threads
    assert lib.starkv_rope_apply(ctypes.byref(d), None) == ERR_LIMIT


def test_cache_writer_limits_and_device_positions():
    lib = L.lib()
    keep = []
    # one wave per row: B * Hkv * T * 64 threads must stay below 2^32
    d = L.KAppendDesc(batch=1 << 14, n_tokens=1 << 12, pos0=0, capacity=1 << 20, dtype=L.F16, src=FAKE,
                      src_stride_b=0, src_stride_h=0, src_stride_t=0, k=_klatent([32] * 8, keep))
    d.pos0_device = FAKE
    assert lib.starkv_k_append(ctypes.byref(d), None) == ERR_LIMIT
    v = L.VAppendDesc(batch=1 << 14, n_tokens=1 << 12, pos0=0, capacity=1 << 20, dtype=L.F16, src=FAKE,
                      src_stride_b=0, src_stride_t=0,
                      v=L.VLatent(rank=1024, format=L.FMT_INT4_G64, data=FAKE, stride_b=0, stride_s=512,
                                  scale=FAKE, scale_stride_b=0, scale_stride_s=16, zero=FAKE))
    v.pos0_device = FAKE
    assert lib.starkv_v_append(ctypes.byref(v), None) == ERR_LIMIT      # 2^26 rows x 16 groups x 64
    # without a device position the host checks the capacity itself
    v.pos0_device, v.batch, v.n_tokens, v.capacity = None, 1, 9, 8
    assert lib.starkv_v_append(ctypes.byref(v), None) == ERR_SHAPE



# ---------------------------------------------------------------- e2e layer ops

def _norm_desc(**kw):
    d = L.RmsNormDesc()
    d.rows, d.hidden, d.dtype = 8, 4096, L.F16
    d.x, d.x_stride, d.weight, d.eps, d.out, d.out_stride = FAKE, 4096, FAKE, 1e-6, FAKE, 4096
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,code", [
    (dict(hidden=4100), ERR_SHAPE), (dict(hidden=16392), ERR_LIMIT), (dict(rows=-1), ERR_SHAPE),
    (dict(dtype=L.F32), ERR_DTYPE), (dict(weight=None), ERR_NULL), (dict(residual_out=FAKE), ERR_NULL),
    (dict(x_stride=4100), ERR_ALIGN), (dict(out=FAKE + 8), ERR_ALIGN), (dict(eps=-1.0), ERR_SHAPE),
    (dict(residual=FAKE, residual_stride=12), ERR_ALIGN),
])
def test_rms_norm_rejects(kw, code):
    assert L.lib().starkv_rms_norm(ctypes.byref(_norm_desc(**kw)), None) == code


@pytest.mark.parametrize("kw,code", [
    (dict(width=12), ERR_SHAPE), (dict(dtype=L.F32), ERR_DTYPE), (dict(up=None), ERR_NULL),
    (dict(gate_stride=22020), ERR_ALIGN), (dict(out=FAKE + 2), ERR_ALIGN),
])
def test_silu_mul_rejects(kw, code):
    d = L.SiluMulDesc()
    d.rows, d.width, d.dtype = 8, 11008, L.F16
    d.gate, d.gate_stride, d.up, d.up_stride, d.out, d.out_stride = FAKE, 22016, FAKE + 22016, 22016, FAKE, 11008
    for k, v in kw.items():
        setattr(d, k, v)
    assert L.lib().starkv_silu_mul(ctypes.byref(d), None) == code


@pytest.mark.parametrize("kw,code", [
    (dict(m=17), ERR_LIMIT), (dict(m=0), ERR_SHAPE), (dict(k=4100), ERR_SHAPE), (dict(k=4128), ERR_SHAPE), (dict(n=4104), ERR_SHAPE),
    (dict(epilogue=3), ERR_SHAPE), (dict(epilogue=2, n=4112), ERR_SHAPE), (dict(dtype=L.F32), ERR_DTYPE),
    (dict(w=None), ERR_NULL), (dict(x_stride=4000), ERR_SHAPE), (dict(out_stride=100), ERR_SHAPE),
    (dict(w_stride=4100), ERR_ALIGN), (dict(x=FAKE + 8), ERR_ALIGN), (dict(out=FAKE + 1), ERR_ALIGN),
])
def test_skinny_gemm_rejects(kw, code):
    d = L.SkinnyGemmDesc()
    d.m, d.n, d.k, d.dtype, d.epilogue = 8, 4096, 4096, L.F16, 0
    d.x, d.x_stride, d.w, d.w_stride, d.out, d.out_stride = FAKE, 4096, FAKE, 4096, FAKE, 4096
    for k, v in kw.items():
        setattr(d, k, v)
    assert L.lib().starkv_skinny_gemm(ctypes.byref(d), None) == code
