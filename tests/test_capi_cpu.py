"""The C-ABI library on the CPU: it loads without a GPU, exports every entry
point include/fireprot_amd.h declares (and the ctypes bindings cover them),
and rejects bad arguments on the host before touching any device pointer
(status 2 sizes/layout, 3 pointers, 4 workspace), as the reference's C ABI
does (kernels/amd/fireprot_ck_attention.cpp:35, 47, 106-108;
tests/operators/test_ck_attention_vector1000.py:16-18).  No call here
reaches a kernel launch."""
from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

from fireprot_amd import _native

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "fireprot_amd.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b((?:fpx|ck)_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        from fireprot_amd import build
        build.build()
    return _native.library()


def test_every_declared_symbol_is_exported_and_bound(lib):
    declared = _declared()
    assert len(declared) >= 10
    raw = ctypes.CDLL(str(_native.LIB_PATH))
    for name in declared:
        assert hasattr(raw, name), f"{name} declared but not exported"
    assert sorted(_native.SIGNATURES) == declared


def test_abi_version_and_workspace_sizes(lib):
    assert lib.fpx_abi_version() == _native.ABI_VERSION == 1
    for n in (1, 124, 512, 1000, 1536, 2048):
        np_ = -(-n // 128) * 128
        seg = lambda b: -(-b // 256) * 256  # noqa: E731
        for dtype, e in ((0, 4), (1, 2)):
            copies = 2 if dtype == 0 else 1  # FP32: unscaled and log2(e)-scaled bias
            # q, k, v^T; gate (rows padded to np); gated output; bias; mask bias;
            # tile flags (4 parts of 4 words per row) plus the 6-word magnitude record;
            # the q, k and v^T tiles' inverse scales of the plane layout; FP32:
            # the constant-mask rows' weights (64 words and two lists of
            # ceil(n / 4) chunk indices, the weight sums [4][np], 4 KB of
            # planes per (head, 32-query tile, 32-key tile))
            expected = (3 * seg(n * 4 * np_ * 32 * e) + seg(n * np_ * 128 * e)
                        + seg(n * n * 128 * e)
                        + seg(4 * np_ * np_ * e * copies) + seg(n * np_ * 4)
                        + seg((n * 16 + 6) * 4) + seg(3 * n * 4 * (np_ // 32) * 4))
            if dtype == 0:
                expected += (seg((64 + 2 * -(-n // 4)) * 4) + seg(4 * np_ * 4)
                             + 4 * (np_ // 32) * (-(-n // 32)) * 4096)
            assert lib.fpx_tri_attn_workspace_bytes(n, 128, 4, 32, dtype) == expected
    for bad in ((0, 128, 4, 32, 0), (4097, 128, 4, 32, 0), (64, 64, 4, 32, 0),
                (64, 128, 8, 32, 0), (64, 128, 4, 16, 0), (64, 128, 4, 32, 7)):
        assert lib.fpx_tri_attn_workspace_bytes(*bad) == 0


def test_strided_workspace_sizes(lib):
    seg = lambda b: -(-b // 256) * 256  # noqa: E731
    for batch, n in ((1, 1), (7, 96), (1536, 1000), (1536, 1536), (3, 4096)):
        np_ = -(-n // 128) * 128
        # two fragment-order bias copies; mask-bias rows; tile flags (4 x 4 words);
        # q, k, v planes (np * 128 bytes per row and head); their scales; the
        # magnitude record (6 words); the staging's per-group maxima
        expected = (2 * seg(4 * np_ * np_ * 4) + seg(batch * np_ * 4) + seg(batch * 16 * 4)
                    + 3 * seg(batch * 4 * np_ * 128) + seg(3 * batch * 4 * (np_ // 32) * 4)
                    + seg(6 * 4) + seg(3 * ((3 * batch * 4 * (np_ // 32) + 3) // 4) * 4))
        assert lib.fpx_attn_strided_workspace_bytes(batch, n) == expected
    for bad in ((0, 8), (2, 0), (2, 4097)):
        assert lib.fpx_attn_strided_workspace_bytes(*bad) == 0


def _strided_args(**override):
    args = dict(q=256, qb=1024, qh=32, qn=128, k=256, kb=1024, kh=32, kn=128, v=256, vb=1024,
                vh=32, vn=128, mask=None, mb=0, mk=1, bias=None, bh=0, bq=0, bk=0, out=512,
                ob=1024, oh=32, on=128, batch=2, n=8, ws=256, ws_bytes=1 << 30, stream=None)
    args.update(override)
    return list(args.values())


def test_strided_guards(lib):
    f = lib.fpx_attn_strided
    assert f(*_strided_args(n=0)) == 2
    assert f(*_strided_args(n=4097)) == 2
    assert f(*_strided_args(batch=0)) == 2
    assert f(*_strided_args(qn=130)) == 2                           # rows not 16-byte aligned
    assert f(*_strided_args(kh=-32)) == 2
    assert f(*_strided_args(vn=1 << 30, n=4096)) == 2               # (b, h) slice beyond 2 GiB
    assert f(*_strided_args(mk=-1)) == 2
    assert f(*_strided_args(bq=-1)) == 2
    assert f(*_strided_args(q=None)) == 3
    assert f(*_strided_args(out=260)) == 3
    assert f(*_strided_args(mask=2)) == 3
    assert f(*_strided_args(bias=6)) == 3
    assert f(*_strided_args(ws=128)) == 3
    assert f(*_strided_args(ws_bytes=1)) == 4


def test_tri_mul_workspace_sizes(lib):
    seg = lambda b: -(-b // 256) * 256  # noqa: E731
    for n in (1, 7, 129, 1000, 1536, 4096):
        np_ = -(-n // 128) * 128
        # a and b channel-major [128][np][np]; x blocked [n][np/32][128][32];
        # the row maxima of a and b [2][128][np] uint32
        expected = 2 * seg(128 * np_ * np_ * 4) + seg(n * np_ * 128 * 4) + seg(2 * 128 * np_ * 4)
        assert lib.fpx_tri_mul_workspace_bytes(n, 128, 128) == expected
    for bad in ((0, 128, 128), (4097, 128, 128), (64, 64, 128), (64, 128, 32)):
        assert lib.fpx_tri_mul_workspace_bytes(*bad) == 0


def _tri_mul_args(**override):
    args = dict(z=256, zs0=64 * 128, zs1=128, mask=None, ms0=0, ms1=0, ln_in_w=None,
                ln_in_b=None, eps_in=1e-5, w=256, b=None, ln_out_w=None, ln_out_b=None,
                eps_out=1e-5, w_z=256, b_z=None, w_g=256, b_g=None, n=64, c_z=128, c_h=128,
                outgoing=1, accumulate=0, out=512, os0=64 * 128, os1=128, ws=256, ws_bytes=1,
                stream=None)
    args.update(override)
    return list(args.values())


def test_tri_mul_guards(lib):
    f = lib.fpx_tri_mul
    assert f(*_tri_mul_args()) == 4                                 # workspace too small
    assert f(*_tri_mul_args(n=0)) == 2
    assert f(*_tri_mul_args(n=4097)) == 2
    assert f(*_tri_mul_args(c_h=64)) == 2
    assert f(*_tri_mul_args(outgoing=2)) == 2
    assert f(*_tri_mul_args(accumulate=-1)) == 2
    assert f(*_tri_mul_args(zs1=130)) == 2                          # rows not 16-byte aligned
    assert f(*_tri_mul_args(os0=-1)) == 2
    assert f(*_tri_mul_args(mask=256, ms1=-1)) == 2
    assert f(*_tri_mul_args(eps_out=-1.0)) == 2
    assert f(*_tri_mul_args(out=256, os0=128, os1=64 * 128)) == 2   # z aliased, other strides
    assert f(*_tri_mul_args(z=None)) == 3
    assert f(*_tri_mul_args(z=260)) == 3
    assert f(*_tri_mul_args(w_g=None)) == 3
    assert f(*_tri_mul_args(mask=2)) == 3
    assert f(*_tri_mul_args(ln_in_w=4)) == 3
    assert f(*_tri_mul_args(ws=128)) == 3


def test_transition_workspace_and_guards(lib):
    for ri, rj in ((1, 1), (3, 5), (1536, 1536), (1, 1000000)):
        # the fused kernel's weight planes, folded biases and plane exponents
        # (16 x 48 KB + 4 KB + 5 KB), whatever the number of rows: the hidden
        # layer h never reaches memory
        expected = 16 * 48 * 1024 + 4096 + 5120
        assert lib.fpx_transition_workspace_bytes(ri, rj, 128, 4) == expected
    for bad in ((0, 5, 128, 4), (5, 0, 128, 4), (2, 2, 64, 4), (2, 2, 128, 2), (-1, 2, 128, 4)):
        assert lib.fpx_transition_workspace_bytes(*bad) == 0
    f = lib.fpx_transition

    def args(**o):
        a = dict(x=256, ri=4, rj=4, xsi=512, xsj=128, ln_w=None, ln_b=None, eps=1e-5, w_a=256,
                 w_b=256, w_o=256, c=128, e=4, acc=0, out=512, osi=512, osj=128, ws=256,
                 ws_bytes=1, stream=None)
        a.update(o)
        return list(a.values())

    assert f(*args()) == 4
    assert f(*args(ri=0)) == 2
    assert f(*args(e=2)) == 2
    assert f(*args(acc=3)) == 2
    assert f(*args(xsj=127)) == 2
    assert f(*args(osi=-1)) == 2
    assert f(*args(eps=-1.0)) == 2
    assert f(*args(out=256, osi=128, osj=512)) == 2     # x aliased with other strides
    assert f(*args(x=None)) == 3
    assert f(*args(w_o=8)) == 3
    assert f(*args(ln_b=4)) == 3
    assert f(*args(ws=128)) == 3


def _block_args(**override):
    args = dict(dtype=0, z=256, zs0=64 * 128, zs1=128, mask=None, ms0=0, ms1=0, ln_w=None,
                ln_b=None, eps=1e-5, w_qkvg=256, b_g=None, w_bias=256, w_o=256, b_o=None,
                inf=1e9, n=64, c=128, heads=4, head_dim=32, ending=0, dz=256, ds0=64 * 128,
                ds1=128, ws=256, ws_bytes=1, stream=None)
    args.update(override)
    return list(args.values())


def test_block_guards(lib):
    f = lib.fpx_tri_attn_block
    assert f(*_block_args()) == 4                                   # workspace too small
    assert f(*_block_args(n=0)) == 2
    assert f(*_block_args(c=64)) == 2
    assert f(*_block_args(dtype=7)) == 2                            # unknown storage type
    assert f(*_block_args(dtype=1)) == 4                            # BF16: workspace too small
    assert f(*_block_args(dtype=1, zs1=132)) == 2                   # bf16 rows need 8-element strides
    assert f(*_block_args(ending=2)) == 2
    assert f(*_block_args(zs1=126)) == 2                            # rows not 16-byte aligned
    assert f(*_block_args(eps=-1.0)) == 2
    assert f(*_block_args(inf=float("inf"))) == 2
    assert f(*_block_args(z=None)) == 3
    assert f(*_block_args(z=260)) == 3
    assert f(*_block_args(w_o=None)) == 3
    assert f(*_block_args(ws=128)) == 3                              # 256-byte workspace
    assert f(*_block_args(mask=2)) == 3
    assert lib.fpx_tri_attn_attend(0, 64, 256, 1, None) == 4
    assert lib.fpx_tri_attn_attend(0, 0, 256, 1, None) == 2
    assert lib.fpx_tri_attn_attend(0, 64, None, 1 << 40, None) == 3


def test_core_and_stage_op_guards(lib):
    core = lib.fpx_attn_core
    assert core(None, None, None, None, None, 1000, 999, None) == 2
    assert core(None, None, None, None, None, 0, 1000, None) == 2
    assert core(None, None, None, None, None, 1000, 1000, None) == 3
    assert core(4, 16, 16, 16, 16, 1000, 1000, None) == 3
    masked = lib.fpx_attn_core_masked
    assert masked(16, 16, 16, None, 0, 16, 1000, 16, 1, 1004, None) == 2   # stride < n
    assert masked(16, 16, 16, None, 0, 16, 1002, 16, 1, 1000, None) == 2   # stride % 4
    assert masked(16, 16, 16, 2, 1000, 16, 1000, 16, 1, 1000, None) == 3   # mask alignment
    ln = lib.fpx_layer_norm_c128
    assert ln(16, -1, 1, 128, 128, None, None, 1e-5, 16, None) == 2
    assert ln(16, 1, 1, 127, 128, None, None, 1e-5, 16, None) == 2
    assert ln(None, 1, 1, 128, 128, None, None, 1e-5, 16, None) == 3
    assert ln(16, 1, 1, 128, 128, 4, None, 1e-5, 16, None) == 3
    qkv = lib.fpx_qkv_projection
    assert qkv(16, -1, 16, 16, 16, 16, None) == 2
    assert qkv(16, 10, 16, None, 16, 16, None) == 3
    sig = lib.fpx_sigmoid_mul_out
    assert sig(16, 16, 16, 6, None) == 2
    assert sig(16, 8, 16, 8, None) == 3


def test_status_errors_raise():
    _native.check(0, "ok")
    for code, word in ((2, "unsupported"), (3, "pointer"), (4, "workspace"), (98, "HIP")):
        with pytest.raises(RuntimeError, match=word):
            _native.check(code, "call")


def test_reference_named_entries_reject_other_shapes_before_touching_memory(lib):
    """ck_attention, ck_attention_exact1536 and ck_attention_vector_bias1000
    accept only their reference shapes (fireprot_ck_attention.cpp:35, 68,
    106) and check pointers before any launch."""
    for name, good in (("ck_attention", ((1000, 1000), (512, 1536))),
                       ("ck_attention_exact1536", ((512, 1536),)),
                       ("ck_attention_vector_bias1000", ((1000, 1000),))):
        fn = getattr(lib, name)
        for batch, n in ((1, 1536), (512, 1000), (1000, 1536), (511, 1536), (1000, 999)):
            if (batch, n) not in good:
                assert fn(None, None, None, None, None, batch, n, None) == 2, (name, batch, n)
        for batch, n in good:
            assert fn(None, None, None, None, None, batch, n, None) == 3, (name, batch, n)
            assert fn(16, 16, 16, 4, 16, batch, n, None) == 3, (name, batch, n)
