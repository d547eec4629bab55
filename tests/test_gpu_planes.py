"""The plane layout the FP32 block's prepare stage writes for its attention.

Per (outer row, head) the workspace holds a hi plane and then a lo plane of
16-bit values.  q and k are [np rows][32 channels] fp16 planes of the value
scaled by a power of two, v^T the same as fp16 planes [key tile][32
channels][32 key positions] with a tile's keys in the S^T accumulator's
register order.  The scale is one per head and operand, from the bound
|x W^T| <= sum_c |W_c| (sqrt(128) |ln_w_c| + |ln_b_c|) that every
LayerNorm-normalised row obeys, so that the bound times the scale lies in
[2^14, 2^15); the workspace keeps the inverse scale for every tile.  Decoding
the planes must give the FP32 projections back to 22 significant bits, every
scaled value must stay below 2^15, and the scales must be the promised
powers of two, equal over every row and tile of a head.  The workspace is filled with NaN bytes
first: every plane row the attention reads, padded rows included, must be
written.  The layout is internal to the block's workspace; the offsets below
restate the workspace segments (capi.hip).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from fireprot_amd import _native
from fireprot_amd import block as hip_block
from fireprot_amd import workloads
from oracle import triangle_attention as oracle
from tests.helpers import oracle_params

pytestmark = pytest.mark.gpu


def _seg(b: int) -> int:
    return -(-b // 256) * 256


def _offsets(n: int) -> dict:
    np_ = -(-n // 128) * 128
    qkv = _seg(n * 4 * np_ * 32 * 4)
    o = {"np": np_, "qh": 0, "kh": qkv, "vt": 2 * qkv, "gs": 3 * qkv}
    o["og"] = o["gs"] + _seg(n * np_ * 128 * 4)
    o["bias"] = o["og"] + _seg(n * n * 128 * 4)
    o["mbias"] = o["bias"] + _seg(4 * np_ * np_ * 4 * 2)
    o["flags"] = o["mbias"] + _seg(n * np_ * 4)
    o["scales"] = o["flags"] + _seg((n * 16 + 6) * 4)
    return o


def _f16(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16).astype(np.float64)


def _key_positions() -> np.ndarray:
    """Position of each key of a 32-key tile in the v^T planes."""
    perm = (0, 2, 1, 3)
    return np.array([16 * (k // 16) + 4 * perm[(k // 4) % 4] + k % 4 for k in range(32)])


@pytest.mark.parametrize("ending", [False, True])
@pytest.mark.parametrize("scale", [1.0, 300.0, 1e-3])
def test_prepare_planes_decode_to_the_projections(ending, scale):
    n = 100
    z = workloads.make_pair(n)
    w = workloads.make_weights()
    for key in ("w_q", "w_k", "w_v"):
        w[key] = w[key] * scale
    # a constant pair row: its normalised row is the LN bias, far smaller
    # than the other rows of its head (far below the head's bound)
    z[3, 7] = 5.0
    weights = hip_block.BlockWeights.from_tensors(**w).to("cuda")
    lib = _native.library()
    ws_bytes = hip_block.workspace_bytes(n, torch.float32)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device="cuda")
    zc = z.cuda()
    code = lib.fpx_tri_attn_prepare(
        0, zc.data_ptr(), zc.stride(0), zc.stride(1), None, 0, 0,
        weights.ln_w.data_ptr() if weights.ln_w is not None else None,
        weights.ln_b.data_ptr() if weights.ln_b is not None else None, weights.eps,
        weights.w_qkvg.data_ptr(), None, weights.w_bias.data_ptr(), weights.inf, n, int(ending),
        ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_tri_attn_prepare")
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    o = _offsets(n)
    np_, nt = o["np"], o["np"] // 32

    def halves(start, count):
        return raw[start:start + 2 * count].view(np.uint16)

    scales = raw[o["scales"]:o["scales"] + 4 * 3 * n * 4 * nt].view(np.float32).reshape(3, n, 4, nt)
    mant, _ = np.frexp(scales)
    assert np.all(mant == 0.5), "scales must be powers of two"
    for op in range(3):  # one scale per head: the same over every row and tile
        per_head = scales[op].transpose(1, 0, 2).reshape(4, -1)
        assert np.all(per_head == per_head[:, :1]), f"operand {op}: scales differ within a head"

    params = oracle_params(w).to(torch.float64)
    x = z.transpose(0, 1) if ending else z
    xl = oracle.layer_norm(x.double(), params.ln_w, params.ln_b, params.eps)
    eq, ek, ev = oracle.prep_qkv(xl, params, apply_scale=True)

    for t, (seg, ref) in enumerate((("qh", eq), ("kh", ek))):
        planes = halves(o[seg], n * 4 * 2 * np_ * 32).reshape(n, 4, 2, np_, 32)
        dec = _f16(planes[:, :, 0]) + _f16(planes[:, :, 1])
        head_max = np.abs(dec).transpose(1, 0, 2, 3).reshape(4, -1).max(axis=-1)
        # below the fp16 range, and within a few binary orders of the bound
        assert np.all((head_max < 2.0 ** 15) & (head_max >= 2.0 ** 8)), head_max
        val = dec * np.repeat(scales[t], 32, axis=-1)[..., None]
        refn = ref.numpy()
        err = np.abs(val[:, :, :n] - refn).max()
        bound = 2e-6 * np.abs(refn).max()
        print(f"{seg} ending={ending} scale={scale}: max|err|={err:.3e} bound={bound:.3e}", flush=True)
        assert err <= bound
        assert np.all(val[:, :, n:] == 0), "padded rows must be zero"
    planes = halves(o["vt"], n * 4 * 2 * np_ * 32).reshape(n, 4, 2, nt, 32, 32)
    dec = _f16(planes[:, :, 0]) + _f16(planes[:, :, 1])      # [n, 4, tile, channel, position]
    head_max = np.abs(dec).transpose(1, 0, 2, 3, 4).reshape(4, -1).max(axis=-1)
    assert np.all((head_max < 2.0 ** 15) & (head_max >= 2.0 ** 8)), head_max
    vt_pos = dec * scales[2][..., None, None]
    vt = vt_pos[..., _key_positions()]                        # key order within each tile
    vt = vt.transpose(0, 1, 3, 2, 4).reshape(n, 4, 32, np_)   # [n, 4, channel, key]
    refv = ev.numpy().transpose(0, 1, 3, 2)
    err = np.abs(vt[..., :n] - refv).max()
    bound = 2e-6 * np.abs(refv).max()
    print(f"v ending={ending} scale={scale}: max|err|={err:.3e} bound={bound:.3e}", flush=True)
    assert err <= bound
    assert np.all(vt[..., n:] == 0), "padded keys must be zero"


def test_mask_rows_flags_and_row_extremes():
    """The mask stage's bias rows and per-row tile flags, against numpy:
    part 0 / 1 / 2 bit t = some key / every key / every key at or below
    -2^29 of 32-key tile t has a nonzero mask bias, keys past n counting as
    -inf; part 3 = the row's largest mask bias and its smallest over the keys
    < n (NaN-propagating).  The attention classifies rows from these words."""
    n = 100
    np_ = 128
    gen = torch.Generator().manual_seed(5)
    mask = (torch.rand(n, n, generator=gen) > 0.3).float()
    mask[5] = 0.0                 # fully masked: -1e9 on every key
    mask[6, :40] = 2.0            # +1e9 on some keys
    mask[7, 33] = float("nan")
    mask[8] = 1.0                 # no mask bias at all
    z = workloads.make_pair(n)
    weights = hip_block.BlockWeights.from_tensors(**workloads.make_weights()).to("cuda")
    lib = _native.library()
    ws_bytes = hip_block.workspace_bytes(n, torch.float32)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device="cuda")
    zc, mc = z.cuda(), mask.cuda()
    code = lib.fpx_tri_attn_prepare(
        0, zc.data_ptr(), zc.stride(0), zc.stride(1), mc.data_ptr(), mc.stride(0), mc.stride(1),
        weights.ln_w.data_ptr() if weights.ln_w is not None else None,
        weights.ln_b.data_ptr() if weights.ln_b is not None else None, weights.eps,
        weights.w_qkvg.data_ptr(), None, weights.w_bias.data_ptr(), weights.inf, n, 0,
        ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_tri_attn_prepare")
    torch.cuda.synchronize()
    o = _offsets(n)
    raw = ws.cpu().numpy()
    mbias = raw[o["mbias"]:o["mbias"] + n * np_ * 4].view(np.float32).reshape(n, np_)
    flags = raw[o["flags"]:o["flags"] + n * 16 * 4].view(np.uint32).reshape(n, 4, 4)

    m = mask.numpy().astype(np.float32)
    with np.errstate(invalid="ignore"):
        want = np.float32(weights.inf) * (m - np.float32(1.0))
    full = np.full((n, np_), -np.inf, dtype=np.float32)
    full[:, :n] = want
    nan = np.isnan(full)
    np.testing.assert_array_equal(np.isnan(mbias), nan)
    np.testing.assert_array_equal(mbias[~nan], full[~nan])
    tiles = full.reshape(n, np_ // 32, 32)
    with np.errstate(invalid="ignore"):
        parts = [(tiles != 0).any(2), (tiles != 0).all(2), (tiles <= -2.0 ** 29).all(2)]
    for p, bits in enumerate(parts):
        words = np.zeros((n, 4), dtype=np.uint64)
        for t in range(np_ // 32):
            words[:, t // 32] |= bits[:, t].astype(np.uint64) << np.uint64(t % 32)
        np.testing.assert_array_equal(flags[:, p, :].astype(np.uint64), words, err_msg=f"part {p}")
    hi = flags[:, 3, 0].view(np.float32)
    lo = flags[:, 3, 1].view(np.float32)
    want_hi = full.max(1)
    want_lo = full[:, :n].min(1)
    for got, exp, name in ((hi, want_hi, "max"), (lo, want_lo, "min")):
        np.testing.assert_array_equal(np.isnan(got), np.isnan(exp), err_msg=name)
        keep = ~np.isnan(exp)
        np.testing.assert_array_equal(got[keep], exp[keep], err_msg=name)
    assert hi[5] == lo[5] == np.float32(-1e9) and hi[8] == lo[8] == 0.0 and np.isnan(hi[7])


def _frag_index(h, q, k, np_):
    """bias_frag_index (common.hpp): fragment-major position of bias[h, q, k]."""
    nt = np_ // 32
    t = k & 31
    return ((((h * nt + (q >> 5)) * nt + (k >> 5)) * 1024) + (t >> 3) * 256
            + ((q & 31) + 32 * ((t >> 2) & 1)) * 4 + (t & 3))


@pytest.mark.parametrize("case", ["tail", "ragged", "first_key_masked"])
def test_relative_log2_bias(case):
    """After the prepare stage the log2-scaled bias copy holds, per query q,
    bias log2(e) - (C_q - 8): C_q the ceiling of q's largest log2 bias over
    the 32-key tiles before T, T the first tile with a nonzero mask bias on
    any row that has an unmasked key; the record's word 5 says so.  With T = 0
    (a row whose first key is masked while others are not) the copy stays
    bias log2(e) and the word stays 0.  Checked bit for bit against numpy on
    the natural-units copy."""
    n = 100
    np_ = 128
    valid = {"tail": [90] * n, "ragged": [40 + (i % 3) * 20 for i in range(n)],
             "first_key_masked": [90] * n}[case]
    mask = torch.zeros(n, n)
    for i, v in enumerate(valid):
        mask[i, :v] = 1.0
    mask[95:] = 0.0  # fully masked rows take no part in T
    if case == "first_key_masked":
        mask[3, 0] = 0.0
    z = workloads.make_pair(n)
    weights = hip_block.BlockWeights.from_tensors(**workloads.make_weights(bias_scale=8.0)).to("cuda")
    lib = _native.library()
    ws_bytes = hip_block.workspace_bytes(n, torch.float32)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device="cuda")
    zc, mc = z.cuda(), mask.cuda()
    code = lib.fpx_tri_attn_prepare(
        0, zc.data_ptr(), zc.stride(0), zc.stride(1), mc.data_ptr(), mc.stride(0), mc.stride(1),
        weights.ln_w.data_ptr(), weights.ln_b.data_ptr(), weights.eps,
        weights.w_qkvg.data_ptr(), None, weights.w_bias.data_ptr(), weights.inf, n, 0,
        ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_tri_attn_prepare")
    torch.cuda.synchronize()
    o = _offsets(n)
    raw = ws.cpu().numpy()
    frags = 4 * np_ * np_
    nat = raw[o["bias"]:o["bias"] + 4 * frags].view(np.float32)
    l2 = raw[o["bias"] + 4 * frags:o["bias"] + 8 * frags].view(np.float32)
    record = raw[o["flags"] + n * 16 * 4:o["flags"] + n * 16 * 4 + 6 * 4].view(np.uint32)
    h, q, k = np.meshgrid(np.arange(4), np.arange(np_), np.arange(np_), indexing="ij")
    idx = _frag_index(h, q, k, np_)
    bias_nat = nat[idx]                                     # [4, np, np]
    log2 = (bias_nat * np.float32(1.4426950408889634)).astype(np.float32)
    first = [min(v, n) // 32 for v in valid[:95]]           # first tile with a masked key
    t_first = 0 if case == "first_key_masked" else min(first)
    got = l2[idx]
    if t_first == 0:
        assert record[5] == 0
        np.testing.assert_array_equal(got, log2)
        return
    assert record[5] == 1
    c = np.ceil(log2[:, :, :32 * t_first].max(axis=2))      # [4, np]
    want = (log2 - (c - np.float32(8.0))[:, :, None].astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n,ending", [(64, False), (100, True), (300, False)])
def test_prepare_magnitude_record(n, ending):
    """The prepare stage's magnitude record holds max |q| (times 1/sqrt(32)),
    max |k|, max |v| and max |triangle bias| over the pair, and its valid
    word.  The attention bounds its logits and picks its softmax path from
    these maxima, so each must be the projections' own maximum: each work-group
    combines its waves' maxima before one atomic per word, and at N=64
    every work-group holds a single tile and all finish together."""
    z = workloads.make_pair(n)
    w = workloads.make_weights(bias_scale=8.0)
    weights = hip_block.BlockWeights.from_tensors(**w).to("cuda")
    lib = _native.library()
    ws_bytes = hip_block.workspace_bytes(n, torch.float32)
    ws = torch.full((ws_bytes,), 0xFF, dtype=torch.uint8, device="cuda")
    zc = z.cuda()
    code = lib.fpx_tri_attn_prepare(
        0, zc.data_ptr(), zc.stride(0), zc.stride(1), None, 0, 0,
        weights.ln_w.data_ptr(), weights.ln_b.data_ptr(), weights.eps,
        weights.w_qkvg.data_ptr(), None, weights.w_bias.data_ptr(), weights.inf, n, int(ending),
        ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_tri_attn_prepare")
    torch.cuda.synchronize()
    o = _offsets(n)
    raw = ws.cpu().numpy()
    words = raw[o["flags"] + n * 16 * 4:o["flags"] + n * 16 * 4 + 5 * 4]
    record = words.view(np.float32)
    assert words.view(np.uint32)[4] == 1

    params = oracle_params(w).to(torch.float64)
    x = z.transpose(0, 1) if ending else z
    xl = oracle.layer_norm(x.double(), params.ln_w, params.ln_b, params.eps)
    eq, ek, ev = oracle.prep_qkv(xl, params, apply_scale=True)
    bias = oracle.triangle_bias(xl, params)
    want = [float(t.abs().max()) for t in (eq, ek, ev, bias)]
    for name, got, ref in zip(("q", "k", "v", "bias"), record[:4], want):
        print(f"n={n} ending={ending} max|{name}|: record {got:.9g}, float64 {ref:.9g}", flush=True)
        assert abs(float(got) - ref) <= 1e-5 * ref, name
