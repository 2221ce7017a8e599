"""Independent pins of the oracle's quantizers, epilogues and matmuls.

Each check restates the function with numpy / torch arithmetic chosen so
that a plausible slip in the oracle -- a wrong divisor (/127 for /448), a
dropped bias or residual term, a transposed operand, a different operation
order (acc * (s_in * s_w) against (acc * s_in) * s_w), a wrong rounding mode
-- fails it:

* fused multiply-adds are emulated exactly in float64 (the product of two
  float32 values is exact in float64; the sum is then rounded once to
  float32, which differs from a true fma only when the float64 sum itself
  was rounded onto a float32 tie -- probability ~2^-29 per value);
* e4m3 encodings come from torch.float8_e4m3fn (round to nearest even),
  after clamping to +-448 because the oracle saturates;
* integer rounding is numpy's rint (ties to even);
* matmuls are float64 numpy / exact int64.
The reference lines each function restates are cited in the oracle.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

F32 = np.float32


def f32_fma(a, b, c):
    """fmaf(a, b, c) for float32 arrays (see the module docstring)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F32)


def e4m3(values):
    v = torch.from_numpy(np.clip(np.asarray(values, F32), -448.0, 448.0))
    return v.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def f16_bits(values):
    return np.asarray(values, F32).astype(np.float16).view(np.uint16)


def acts(m, k, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * scale).astype(np.float16)
    x[0, :7] = np.array([0, -0.0, 65504, -65504, 6e-8, -6e-8, 1.0], np.float16)
    if m > 2:
        x[2] = 0  # an all-zero row
    return x


# ---- static quantizers (linear.cu:537-560) ---------------------------------------------

def test_quantize_fp8_static_matches_torch(oracle):
    x = acts(64, 256, 1)
    for inv in (1.0, 56.0, 1.0 / 3.0, 3.7e-3, 448.0 / 0.125):
        ref = e4m3(x.astype(F32) * F32(inv))
        assert np.array_equal(oracle.quantize_fp8_static(x, inv), ref), inv


def test_quantize_int8_static_matches_numpy(oracle):
    x = acts(64, 256, 2)
    # exact halves exercise the ties-to-even rule
    x[1, :8] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float16)
    for inv in (1.0, 127.0 / 8.0, 0.37):
        s = x.astype(F32) * F32(inv)
        ref = np.rint(np.clip(s, -127.0, 127.0)).astype(np.int8)
        assert np.array_equal(oracle.quantize_int8_static(x, inv), ref), inv


# ---- dynamic per-row quantizers (encoder.cu:264-292, 1129-1180) -----------------------

def test_quantize_fp8_rows_matches_torch(oracle):
    x = acts(40, 512, 3)
    q, s = oracle.quantize_fp8_rows(x, valid_rows=37)
    m = np.abs(x.astype(F32)).max(axis=1)
    scale = np.where(m > 0, m / F32(448.0), F32(1.0)).astype(F32)
    scale[37:] = 1.0
    ref = e4m3(x.astype(F32) / scale[:, None])
    ref[37:] = 0
    assert np.array_equal(s, scale)
    assert np.array_equal(q, ref)


def test_quantize_int8_rows_matches_numpy(oracle):
    x = acts(40, 512, 4)
    q, s = oracle.quantize_int8_rows(x, valid_rows=39)
    m = np.abs(x.astype(F32)).max(axis=1)
    scale = np.where(m > 0, m / F32(127.0), F32(1.0)).astype(F32)
    scale[39:] = 1.0
    ref = np.clip(np.rint(x.astype(F32) / scale[:, None]), -127, 127).astype(np.int8)
    ref[39:] = 0
    assert np.array_equal(s, scale)
    assert np.array_equal(q, ref)


def test_quantize_int4_rows_matches_numpy(oracle):
    x = acts(40, 512, 5)
    x[3] = np.abs(x[3])    # positive-only row: the scale is max / 7
    x[4] = -np.abs(x[4])   # negative-only row: the scale is -min / 8
    q, s = oracle.quantize_int4_rows(x, valid_rows=38)
    xf = x.astype(F32)
    m = np.maximum(xf / F32(7.0), -xf / F32(8.0)).max(axis=1)
    scale = np.where(m > 0, m, F32(1.0)).astype(F32)
    scale[38:] = 1.0
    lv = np.clip(np.rint(xf / scale[:, None]), -8, 7).astype(np.int64)
    lv[38:] = 0
    ref = ((lv[:, 0::2] & 15) | ((lv[:, 1::2] & 15) << 4)).astype(np.uint8)
    assert np.array_equal(s, scale)
    assert np.array_equal(q, ref)
    # the negative-only row reaches the level -8
    assert (lv[4] == -8).any()


# ---- epilogues ------------------------------------------------------------------------------

def _acc(m, n, seed, integer=False):
    rng = np.random.default_rng(seed)
    if integer:
        return rng.integers(-200000, 200000, (m, n)).astype(F32)
    return (rng.standard_normal((m, n)) * 40).astype(F32)


@pytest.mark.parametrize("act", [0, 2])
def test_epilogue_quantized_matches_fma_order(oracle, act):
    """linear.cu:362-373 / 417-428: fp16(act(fmaf(acc, s_in * s_w[c], b[c])))."""
    m, n = 512, 1024
    acc = _acc(m, n, 6, integer=True)
    rng = np.random.default_rng(7)
    ws = rng.uniform(1e-4, 2e-3, n).astype(F32)
    bias = (rng.standard_normal(n) * 0.3).astype(F32)
    in_scale = 0.0371
    scale = F32(in_scale) * ws
    v = f32_fma(acc, scale[None, :], bias[None, :])
    if act == 2:
        v = np.maximum(v, F32(0.0))
    got = oracle.epilogue_quantized(acc, in_scale, ws, bias, act)
    assert np.array_equal(got.view(np.uint16), f16_bits(v))
    # no bias: fmaf(acc, s, 0) is one rounding of the product
    got0 = oracle.epilogue_quantized(acc, in_scale, ws, None, 0)
    assert np.array_equal(got0.view(np.uint16), f16_bits(f32_fma(acc, scale[None, :], 0.0)))


def test_epilogue_quantized_silu(oracle):
    m, n = 64, 256
    acc = _acc(m, n, 8, integer=True)
    ws = np.random.default_rng(9).uniform(1e-4, 2e-3, n).astype(F32)
    v = f32_fma(acc, (F32(0.05) * ws)[None, :], 0.0)
    ref = torch.nn.functional.silu(torch.from_numpy(v).double()).numpy()
    got = oracle.epilogue_quantized(acc, 0.05, ws, None, 1).astype(np.float64)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3)) <= 2 ** -10


@pytest.mark.parametrize("act", [0, 2])
def test_epilogue_linear_matches_reference_order(oracle, act):
    """linear.cu:130-147: v = acc (+ bias); v *= out_scale; v = fmaf(res_scale,
    residual, v); act; fp16."""
    m, n = 256, 640
    acc = _acc(m, n, 10)
    rng = np.random.default_rng(11)
    bias = (rng.standard_normal(n) * 0.5).astype(F32)
    res = (rng.standard_normal((m, n)) * 4).astype(np.float16)
    out_scale, res_scale = 0.5, 0.25
    v = (acc + bias[None, :]).astype(F32) * F32(out_scale)
    v = f32_fma(F32(res_scale), res.astype(F32), v)
    if act == 2:
        v = np.maximum(v, F32(0.0))
    got = oracle.epilogue_linear(acc, bias, res, out_scale, res_scale, act)
    assert np.array_equal(got.view(np.uint16), f16_bits(v))
    got = oracle.epilogue_linear(acc, None, None, 1.0, 0.0, 0)
    assert np.array_equal(got.view(np.uint16), f16_bits(acc))


@pytest.mark.parametrize("mode", [2, 3, 4, 6])
def test_ffn_epilogue_modes(oracle, mode):
    """encoder.cu:975-1030: v = (acc * s_row) * s_w; mode 2 fp16(fmaf(0.5, v,
    r)), 3 fp16(v + b), 4 fp16(relu(v + b)), 6 fp16(fmaf(1, v, r))."""
    m, n = 256, 512
    acc = _acc(m, n, 12, integer=True)
    rng = np.random.default_rng(13)
    rs = rng.uniform(1e-3, 1e-2, m).astype(F32)
    ws = rng.uniform(1e-3, 1e-2, n).astype(F32)
    bias = (rng.standard_normal(n) * 0.5).astype(F32)
    res = (rng.standard_normal((m, n)) * 2).astype(np.float16)
    v = (acc * rs[:, None]).astype(F32) * ws[None, :]
    if mode == 2:
        ref = f32_fma(0.5, v, res.astype(F32))
    elif mode == 6:
        ref = f32_fma(1.0, v, res.astype(F32))
    elif mode == 3:
        ref = v + bias[None, :]
    else:
        ref = np.maximum(v + bias[None, :], F32(0.0))
    got = oracle.epilogue(acc, mode, ws, row_scales=rs, bias=bias, residual=res)
    assert np.array_equal(got.view(np.uint16), f16_bits(ref))


def test_ffn_epilogue_e4m3(oracle):
    """encoder.cu:1010-1025: e4m3(fp16(silu(v)) * 16)."""
    m, n = 128, 512
    acc = _acc(m, n, 14, integer=True)
    rng = np.random.default_rng(15)
    rs = rng.uniform(1e-3, 1e-2, m).astype(F32)
    ws = rng.uniform(1e-3, 1e-2, n).astype(F32)
    v = (acc * rs[:, None]).astype(F32) * ws[None, :]
    silu = torch.nn.functional.silu(torch.from_numpy(v).double()).numpy()
    ref = e4m3(silu.astype(np.float16).astype(F32) * F32(16.0))
    got = oracle.epilogue(acc, 1, ws, row_scales=rs)
    # the float64 SiLU may sit on the other side of an fp16 rounding boundary
    # than the oracle's float32 one for a few values: at most one e4m3 code
    assert np.mean(got == ref) > 0.995
    t = oracle.e4m3_table().astype(np.float64)
    assert np.all(np.abs(t[got] - t[ref]) <= np.abs(t[ref]) / 8 + 2.0 ** -9)


# ---- matmuls ----------------------------------------------------------------------------

def _bound(x, w):
    """|fp32 k-order sum - exact| <= k * 2^-24 * sum_k |x_k w_k| (plus slack)."""
    k = x.shape[1]
    return (k * 2.0 ** -24) * (np.abs(x) @ np.abs(w).T) + 1e-30


def test_gemm_f16_matches_float64(oracle):
    rng = np.random.default_rng(16)
    x = (rng.standard_normal((24, 512)) * 2).astype(np.float16)
    w = (rng.standard_normal((40, 512)) * 0.05).astype(np.float16)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    got = oracle.gemm_f16(x, w).astype(np.float64)
    assert np.all(np.abs(got - ref) <= _bound(x.astype(np.float64), w.astype(np.float64)))
    # an operand-order slip (x against w's transpose rows) is far outside it
    assert np.max(np.abs(got - ref)) < 0.01 * np.max(np.abs(ref))


def test_gemm_q4k_matches_float64_of_dequantized(oracle):
    rng = np.random.default_rng(17)
    w = (rng.standard_normal((16, 512)) * 0.05).astype(np.float16)
    blocks = oracle.q4k_encode(w)
    wd = oracle.q4k_dequant(blocks).astype(np.float16).astype(np.float64)  # f16(dequant) (linear.cu:446-457)
    x = (rng.standard_normal((12, 512))).astype(np.float16)
    ref = x.astype(np.float64) @ wd.T
    got = oracle.gemm_q4k(x, blocks).astype(np.float64)
    assert np.all(np.abs(got - ref) <= _bound(x.astype(np.float64), wd))


def test_gemm_g128_a8_fold_order(oracle):
    """out = fold over groups of fmaf(float(group sum), s_g, total), then
    total * x_scale: emulated exactly."""
    rng = np.random.default_rng(18)
    w = (rng.standard_normal((24, 512)) * 0.02).astype(np.float16)
    q, s, z = oracle.pack_int4_g128(w)
    x = (rng.standard_normal((9, 512)) * 2).astype(np.float16)
    x8, xs = oracle.quantize_int8_rows(x)
    out, gacc = oracle.gemm_g128_a8(x8, xs, q, s, z, want_group_acc=True)
    total = np.zeros((9, 24), F32)
    for g in range(4):
        total = f32_fma(gacc[:, :, g].astype(F32), s[:, g].astype(F32)[None, :], total)
    assert np.array_equal(out, total * xs[:, None])


def test_gemm_g128_a8_parts_association(oracle):
    """parts > 1: each contiguous run of groups folded from 0 in order, the run
    sums added in order (the association of the split-K kernel), emulated
    exactly for 2 and 4 runs of 4 groups; 3 runs of 4 groups: runs [0,1),
    [1,2), [2,4)."""
    rng = np.random.default_rng(21)
    w = (rng.standard_normal((24, 512)) * 0.02).astype(np.float16)
    q, s, z = oracle.pack_int4_g128(w)
    x = (rng.standard_normal((9, 512)) * 2).astype(np.float16)
    x8, xs = oracle.quantize_int8_rows(x)
    _, gacc = oracle.gemm_g128_a8(x8, xs, q, s, z, want_group_acc=True)
    for parts, runs in ((2, [(0, 2), (2, 4)]), (4, [(0, 1), (1, 2), (2, 3), (3, 4)]), (3, [(0, 1), (1, 2), (2, 4)])):
        total = None
        for lo, hi in runs:
            part = np.zeros((9, 24), F32)
            for g in range(lo, hi):
                part = f32_fma(gacc[:, :, g].astype(F32), s[:, g].astype(F32)[None, :], part)
            total = part if total is None else (total + part).astype(F32)
        out = oracle.gemm_g128_a8(x8, xs, q, s, z, parts=parts)
        assert np.array_equal(out, total * xs[:, None]), parts


def test_joint_scores_i8_matches_float64(oracle):
    """score[o] = w_scale[o] * sum_k W[o,k] relu(f32(enc_k) + pred_k) + b[o]."""
    rng = np.random.default_rng(19)
    o, h = 1030, 640
    w = rng.integers(-127, 128, (o, h)).astype(np.int8)
    ws = rng.uniform(1e-4, 1e-2, o).astype(F32)
    bias = rng.standard_normal(o).astype(F32)
    enc = rng.standard_normal(h).astype(np.float16)
    pred = rng.standard_normal(h).astype(F32)
    x = np.maximum(enc.astype(F32) + pred, F32(0.0)).astype(np.float64)
    ref = ws.astype(np.float64) * (w.astype(np.float64) @ x) + bias
    got = oracle.joint_scores_i8(w, ws, bias, enc, pred)
    assert np.allclose(got, ref, rtol=2e-7, atol=2e-7 * np.abs(ref).max())
    # the relu is on (enc + pred), not on each term
    bad = ws.astype(np.float64) * (w.astype(np.float64) @ (np.maximum(enc.astype(np.float64), 0) + pred)) + bias
    assert not np.allclose(got, bad, rtol=1e-3)


def test_ffn_epilogue_static_int8(oracle):
    """Mode 9: rint(clip(fp16(silu(v)) * 16, +-127)) -- the static INT8
    quantizer of linear.cu:549-560 on the x16 FF hidden."""
    m, n = 128, 512
    acc = _acc(m, n, 24, integer=True)
    rng = np.random.default_rng(25)
    rs = rng.uniform(1e-3, 1e-2, m).astype(F32)
    ws = rng.uniform(1e-3, 3e-2, n).astype(F32)
    v = (acc * rs[:, None]).astype(F32) * ws[None, :]
    silu = torch.nn.functional.silu(torch.from_numpy(v).double()).numpy()
    ref = np.rint(np.clip(silu.astype(np.float16).astype(F32) * F32(16.0), -127, 127)).astype(np.int8)
    got = oracle.epilogue(acc, 9, ws, row_scales=rs).view(np.int8)
    assert np.mean(got == ref) > 0.995
    assert np.all(np.abs(got.astype(np.int32) - ref) <= 1)
    assert (np.abs(ref) == 127).any() and (ref < 0).any()  # both clamps and SiLU's negative lobe reached


def test_gemm_g128_f8_matches_float64(oracle):
    """e4m3 x INT4-g128: the float64 matmul of the decoded e4m3 activations and
    the dequantized weights (q - z) * s agrees to fp32 rounding of the group
    sums and the folds; a dropped zero point or a wrong group's scale does not."""
    rng = np.random.default_rng(26)
    w = (rng.standard_normal((24, 512)) * 0.02).astype(np.float16)
    q, s, z = oracle.pack_int4_g128(w)
    x8 = e4m3(rng.standard_normal((9, 512)) * 2)
    xf = oracle.e4m3_table()[x8].astype(np.float64)
    b = q.view(np.uint8).reshape(24, -1, 4).astype(np.int64)
    lv = np.concatenate([b & 15, b >> 4], axis=2).reshape(24, -1)
    g = np.arange(512) // 128
    wd = (lv - z.astype(np.float64)[:, g]) * s.astype(np.float64)[:, g]
    ref = xf @ wd.T
    got = oracle.gemm_g128_f8(x8, q, s, z).astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.sqrt(np.mean(ref ** 2))
    wrong = xf @ (lv * s.astype(np.float64)[:, g]).T
    assert np.max(np.abs(got - wrong)) > 1e-2 * np.sqrt(np.mean(ref ** 2))
