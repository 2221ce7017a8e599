"""Pins of the attention oracle (oracle/pk_oracle.c, encoder.cu:561-634 and
:1476-2097) and host-side validation of the attention entry points.

The reference ships no tests or vectors for this path, so the oracle is pinned
by what the mathematics and the published MMA fragment layouts fix:
  * packer byte orders against the PTX ISA fragment tables of
    mma.m16n8k32 .s8 and mma.m16n8k64 .s4 (B operand: thread c of a group holds
    k = 4c..4c+3, 16+4c..16+4c+3, resp. 8c..8c+7, 32+8c..32+8c+7), which the
    reference kernels read 8 bytes per thread at 8c;
  * quantizer scales and round trips (closed form), torch's float8_e4m3fn for
    the FP8 copy of V;
  * both attention kernels against a float64 local relative-position
    attention (softmax((q+u).k + (q+v).p) / sqrt(128)) . V over the 257-key
    window), the packed tile path additionally against the same formula on
    its dequantized operands with U4 probabilities, where the only remaining
    error is the e4m3 output rounding.  Removing the position term from the
    float64 formula makes each of these checks fail by a wide margin.
"""
import ctypes
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "l4-parakeet-rs_amd", "build", "libpk_linear.so")
T = 1040


@pytest.fixture(scope="module")
def orc(oracle):
    oracle.set_threads(8)
    return oracle


def make_inputs(seed, rows, q_gain=1.0):
    rng = np.random.default_rng(seed)
    q = (q_gain * rng.standard_normal((rows, 1024))).astype(np.float16)
    k = rng.standard_normal((rows, 1024)).astype(np.float16)
    v = rng.standard_normal((rows, 1024)).astype(np.float16)
    pos = rng.standard_normal((8 * 272, 128)).astype(np.float16)
    bu = (0.1 * rng.standard_normal(1024)).astype(np.float16)
    bv = (0.1 * rng.standard_normal(1024)).astype(np.float16)
    return q, k, v, pos, bu, bv


def textbook(q, k, v, pos, bu, bv, rows_sel, valid, position_term=True):
    """float64 local relative-position attention, window 128/128."""
    qf, kf, vf = (a.astype(np.float64) for a in (q, k, v))
    pf = pos.astype(np.float64).reshape(8, 272, 128)
    out = np.zeros((len(rows_sel), 1024))
    for ii, r in enumerate(rows_sel):
        keys = np.arange(max(0, r - 128), min(valid - 1, r + 128) + 1)
        for h in range(8):
            sl = slice(128 * h, 128 * h + 128)
            s = kf[keys][:, sl] @ (qf[r, sl] + bu[sl].astype(np.float64))
            if position_term:
                s = s + pf[h][128 - r + keys] @ (qf[r, sl] + bv[sl].astype(np.float64))
            s = s / np.sqrt(128.0)
            p = np.exp(s - s.max())
            out[ii, sl] = (p / p.sum()) @ vf[keys][:, sl]
    return out


def rel_rms(x, ref):
    return float(np.sqrt(((x - ref) ** 2).mean() / (ref ** 2).mean()))


# ---- packer layouts ------------------------------------------------------------


def test_score_vector_layout_is_the_s8_fragment_order(orc):
    onehot = np.eye(128, dtype=np.float16)
    out, sc = orc.pack_score_vectors(onehot)
    out = out.reshape(128, 128)
    for d in range(128):
        chunk, r = divmod(d, 32)
        i, rr = divmod(r, 16)
        c, j = divmod(rr, 4)
        expect = 32 * chunk + 8 * c + 4 * i + j
        nz = np.flatnonzero(out[d])
        assert nz.tolist() == [expect], (d, nz, expect)
        assert out[d, expect] == 127 and sc[d] == np.float32(1.0) / np.float32(127.0)


def test_key_int4_layout_is_the_s4_fragment_order(orc):
    onehot = -np.eye(128, dtype=np.float16)
    out, sc = orc.pack_key_int4(onehot)
    out = out.reshape(128, 64)
    nib = np.stack([out & 15, out >> 4], -1).reshape(128, 128)
    for d in range(128):
        chunk, r = divmod(d, 64)
        i, rr = divmod(r, 32)
        c, n = divmod(rr, 8)
        expect = 2 * (32 * chunk + 8 * c + 4 * i) + n
        nz = np.flatnonzero(nib[d])
        assert nz.tolist() == [expect], (d, nz, expect)
        assert nib[d, expect] == 9  # -7 & 15
        assert sc[d] == np.float32(1.0) / np.float32(7.0)


def _unpack_score(out):
    by = np.array([orc_byte(d) for d in range(128)])
    return out.reshape(-1, 128)[:, by].view(np.int8)


def orc_byte(d):
    lane = d // 4
    return (lane // 8) * 32 + (lane % 4) * 8 + (lane & 4) + d % 4


@pytest.mark.parametrize("int4", [False, True])
def test_packers_round_trip(orc, int4):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 128)) * np.exp(rng.standard_normal((64, 1)))).astype(np.float16)
    x[5] = 0
    if int4:
        out, sc = orc.pack_key_int4(x)
        nibs = np.stack([out.reshape(64, 64) & 15, out.reshape(64, 64) >> 4], -1).reshape(64, 128)
        order = np.array([orc.lib().orc_key_int4_nibble(d) for d in range(128)])
        q = nibs[:, order].astype(np.int64)
        q = np.where(q >= 8, q - 16, q)
        lim = 7
    else:
        out, sc = orc.pack_score_vectors(x)
        q = out.reshape(64, 128)[:, [orc_byte(d) for d in range(128)]].view(np.int8).astype(np.int64)
        lim = 127
    xf = x.astype(np.float64)
    m = np.abs(xf).max(1)
    assert sc[5] == 1.0 and not q[5].any()
    live = m > 0
    np.testing.assert_allclose(sc[live], (m[live] / lim).astype(np.float32), rtol=1e-7)
    assert (np.abs(q).max(1)[live] == lim).all()
    err = np.abs(q * sc[:, None].astype(np.float64) - xf)
    assert (err <= 0.5 * sc[:, None] * (1 + 1e-5)).all()  # float32 division ties


def test_quantize_value_int4_layout_and_round_trip(orc):
    import torch

    rng = np.random.default_rng(4)
    rows = 64
    vt = np.clip(rng.standard_normal((1024, rows)), -7.5, 7.5).astype(np.float16)
    vt[3] = 0
    out = orc.quantize_value_int4(vt, 56.0)
    el = rows * 1024
    fp8 = out[:el].reshape(1024, rows)
    ref8 = torch.from_numpy(vt.astype(np.float32) * np.float32(56.0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(fp8, ref8)
    s4 = out[el:el + el // 2].reshape(1024, rows // 2)
    nib = np.stack([s4 & 15, s4 >> 4], -1).reshape(1024, rows).astype(np.int64)
    q = np.where(nib >= 8, nib - 16, nib)
    sc = out[el + el // 2:].view(np.float32)
    m = np.abs(vt.astype(np.float64)).max(1)
    assert sc[3] == 1.0 and not q[3].any()
    live = m > 0
    np.testing.assert_allclose(sc[live], (m[live] / 7).astype(np.float32), rtol=1e-7)
    assert np.abs(q).max() <= 7
    err = np.abs(q * sc[:, None].astype(np.float64) - vt.astype(np.float64))
    assert (err <= 0.5 * sc[:, None] * (1 + 1e-5)).all()  # float32 division ties


def test_quantize_value_register_writes_only_the_edges(orc):
    rng = np.random.default_rng(5)
    rows, valid = 1024, 1000
    vt = rng.standard_normal((1024, rows)).astype(np.float16)
    full = orc.quantize_value_int4(vt)
    edge = orc.quantize_value_int4(vt, edge_only=True, valid_rows=valid, fill=0xAB)
    el = rows * 1024
    np.testing.assert_array_equal(edge[el:], full[el:])
    f8, e8 = full[:el].reshape(1024, rows), edge[:el].reshape(1024, rows)
    r = np.arange(rows)
    pair = r & ~1
    written = (pair < 272) | (pair + 1 >= valid - 272)
    np.testing.assert_array_equal(e8[:, written], f8[:, written])
    assert (e8[:, ~written] == 0xAB).all()
    assert written.sum() == 272 + (rows - (valid - 272))


# ---- attention oracle against float64 attention ------------------------------------


@pytest.fixture(scope="module")
def case(orc):
    q, k, v, pos, bu, bv = make_inputs(11, T)
    vf = orc.quantize_value_int4(np.ascontiguousarray(v.T))
    pk, ks = orc.pack_key_int4(k)
    pp, ps = orc.pack_score_vectors(pos)
    packed = orc.local_attention(True, q, k, vf, pos, bu, bv, T, packed_key=pk, key_scales=ks,
                                 packed_position=pp, position_scales=ps)
    tc = orc.local_attention(False, q, k, vf, pos, bu, bv, T)
    return dict(q=q, k=k, v=v, pos=pos, bu=bu, bv=bv, vf=vf, pk=pk, ks=ks, pp=pp, ps=ps, packed=packed, tc=tc)


EDGE = [0, 3, 77, 127, 912, 1000, 1039]   # per-query path (boundary tiles)
INTERIOR = [128, 300, 517, 750, 895]     # tile path


def _fp8_value(c, rows):
    """V as the FP8 copy the per-query and tc paths read: e4m3(v*56) * 8/448."""
    import pk_oracle

    return (pk_oracle.e4m3_to_f32(c["vf"][:T * 1024]).reshape(1024, T).T * (8.0 / 448.0)).astype(np.float64)


def test_tc_attention_matches_float64_attention(case):
    c = case
    v8 = _fp8_value(c, T)
    sel = EDGE + INTERIOR
    ref = textbook(c["q"], c["k"], v8, c["pos"], c["bu"], c["bv"], sel, T)
    out = c["tc"][sel].view(np.float16).astype(np.float64)
    assert rel_rms(out, ref) < 0.03
    wrong = textbook(c["q"], c["k"], v8, c["pos"], c["bu"], c["bv"], sel, T, position_term=False)
    assert rel_rms(out, wrong) > 5 * rel_rms(out, ref)


def test_packed_boundary_rows_match_float64_attention(case, orc):
    c = case
    v8 = _fp8_value(c, T)
    ref = textbook(c["q"], c["k"], v8, c["pos"], c["bu"], c["bv"], EDGE, T)
    out = orc.e4m3_to_f32(c["packed"][EDGE]).reshape(len(EDGE), 1024) / 28.0
    assert rel_rms(out, ref) < 0.05  # e4m3 output rounding
    wrong = textbook(c["q"], c["k"], v8, c["pos"], c["bu"], c["bv"], EDGE, T, position_term=False)
    assert rel_rms(out, wrong) > 5 * rel_rms(out, ref)


def test_packed_tile_matches_attention_on_dequantized_operands(case, orc):
    c = case
    key_nib = np.array([orc.lib().orc_key_int4_nibble(d) for d in range(128)])
    b = c["pk"].reshape(-1, 64)
    kn = (b[:, key_nib // 2] >> (4 * (key_nib & 1))) & 15
    K = (np.where(kn >= 8, kn - 16, kn) * c["ks"][:, None].astype(np.float64)).reshape(T, 8, 128)
    P = (c["pp"].reshape(-1, 128)[:, [orc_byte(d) for d in range(128)]].view(np.int8) *
         c["ps"][:, None].astype(np.float64)).reshape(8, 272, 128)
    s4 = c["vf"][T * 1024:T * 1024 * 3 // 2]
    vsc = c["vf"][T * 1024 * 3 // 2:].view(np.float32).astype(np.float64)
    vn = np.stack([s4 & 15, s4 >> 4], 1).reshape(1024, T).astype(np.int64)
    V = (np.where(vn >= 8, vn - 16, vn) * vsc[:, None]).T

    def quant(x, lim):
        m = np.float32(np.abs(x).max())
        s = m / np.float32(lim) if m > 0 else np.float32(1)
        return np.rint(x / s) * np.float64(s)

    def ref(position_term):
        out = np.zeros((len(INTERIOR), 1024))
        for ii, r in enumerate(INTERIOR):
            keys = np.arange(r - 128, r + 129)
            for h in range(8):
                sl = slice(128 * h, 128 * h + 128)
                qq = c["q"][r, sl].astype(np.float32)
                qu = quant((qq + c["bu"][sl].astype(np.float32)).astype(np.float16).astype(np.float32), 7)
                qv = quant((qq + c["bv"][sl].astype(np.float32)).astype(np.float16).astype(np.float32), 127)
                s = K[keys, h] @ qu + (P[h][keys - r + 128] @ qv if position_term else 0)
                e = np.exp(s / np.sqrt(128.0) - (s / np.sqrt(128.0)).max())
                p = np.rint(e * 15) / (15 * e.sum())
                out[ii, sl] = p @ V[keys][:, sl]
        return out

    out = orc.e4m3_to_f32(c["packed"][INTERIOR]).reshape(len(INTERIOR), 1024) / 28.0
    good = rel_rms(out, ref(True))
    assert good < 0.05  # e4m3 output rounding and bf16 scores only
    assert rel_rms(out, ref(False)) > 5 * good
    # The whole approximation (INT4 keys, U4 probabilities, S4 V) stays bounded.
    assert rel_rms(out, textbook(c["q"], c["k"], c["v"], c["pos"], c["bu"], c["bv"], INTERIOR, T)) < 0.4


def test_rows_beyond_rows_and_valid_rows_are_zero(orc):
    rows, valid, padded = 1000, 980, 1024
    q, k, v, pos, bu, bv = make_inputs(12, padded)
    vf = orc.quantize_value_int4(np.ascontiguousarray(v.T))
    pk, ks = orc.pack_key_int4(k)
    pp, ps = orc.pack_score_vectors(pos)
    for packed in (True, False):
        out = orc.local_attention(packed, q, k, vf, pos, bu, bv, rows, valid_rows=valid, packed_key=pk,
                                  key_scales=ks, packed_position=pp, position_scales=ps,
                                  out=np.full((padded, 1024), 0x55, np.uint8 if packed else np.uint16))
        assert not out[valid:].any()
        assert out[:valid].any()


# ---- host validation of the attention entry points (no GPU call is made) ---------------


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libpk_linear.so is not built (run __graft_entry__.build())")
    return ctypes.CDLL(LIB)


def _packed(lib, rows, padded, valid, left, right, stride, align=0):
    fn = lib.pk_local_relpos_attention_packed
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int32] * 6 + [ctypes.c_void_p] * 5
    p = ctypes.c_void_p(0x10000 + align)
    return fn(p, p, None, p, p, p, p, p, rows, padded, valid, left, right, stride, p, p, p, p, None)


def test_attention_rejects_bad_shapes(lib):
    assert _packed(lib, 1040, 1040, 1040, 64, 128, 1040) == -1
    assert _packed(lib, 1040, 1032, 1032, 128, 128, 1032) == -1
    assert _packed(lib, 1041, 1040, 1040, 128, 128, 1040) == -1
    assert _packed(lib, 1040, 1040, 1040, 128, 128, 1024) == -1
    assert _packed(lib, 1040, 1040, 0, 128, 128, 1040) == -1
    assert _packed(lib, 1040, 1040, 1040, 128, 128, 1040, align=8) == -2


def test_value_quantizer_rejects_ragged_rows(lib):
    fn = lib.pk_quantize_value_int4_register
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_float, ctypes.c_int32, ctypes.c_void_p]
    p = ctypes.c_void_p(0x10000)
    assert fn(p, p, 1024 * 8, 56.0, 8, None) == -1
    assert fn(p, p, 1024 * 16, 56.0, 17, None) == -1


# ---- short-form attention and attention-side layouts (encoder.cu:644-671, 1321-1461) ----


def test_quantize_fp8_transpose_against_torch(orc):
    """e4m3 of x * s (torch float8_e4m3fn, RNE, in range), transposed."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    rows = 77
    x = (rng.standard_normal((rows, 1024)) * 3).astype(np.float16)
    x[5, :8] = [0, -0.0, 1e-4, -1e-4, 7.9, -7.9, 0.015625, 2.0 ** -10]
    assert np.abs(x.astype(np.float32) * 16).max() < 448
    out = orc.quantize_fp8_transpose(x, 16.0)
    ref = torch.from_numpy(x.astype(np.float32) * np.float32(16.0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(out, ref.T)


def test_pack_position_heads_is_the_head_major_reshape(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((272, 1024)).astype(np.float16)
    out = orc.pack_position_heads(x)
    np.testing.assert_array_equal(out, x.reshape(272, 8, 128).transpose(1, 0, 2))


@pytest.mark.parametrize("rows,valid", [(300, 300), (300, 260), (64, 64)])
def test_short_attention_matches_float64_attention(orc, rows, valid):
    padded = (rows + 15) // 16 * 16
    q, k, v, pos, bu, bv = make_inputs(23 + rows, padded)
    out = orc.local_attention_short(q, k, v, pos, bu, bv, rows, valid_rows=valid)
    live = min(rows, valid)
    assert not out[live:].view(np.uint16).any()
    sel = sorted({0, 1, live // 2, live - 1, min(live - 1, 130)})
    ref = textbook(q, k, v, pos, bu, bv, sel, valid)
    got = out[sel].astype(np.float64)
    # fp16 output: error within half an fp16 ulp plus the float score / softmax rounding
    assert np.abs(got - ref).max() <= 1e-3 * np.sqrt((ref ** 2).mean()) + np.abs(ref).max() * 2.0 ** -11
    wrong = textbook(q, k, v, pos, bu, bv, sel, valid, position_term=False)
    assert rel_rms(got, wrong) > 100 * rel_rms(got, ref)


def test_short_attention_rejects_bad_shapes(lib):
    P = ctypes.c_void_p
    fn = lib.pk_local_relpos_attention
    fn.argtypes = [P] * 7 + [ctypes.c_int] * 5 + [P]
    fn.restype = ctypes.c_int
    buf = ctypes.create_string_buffer(64)
    a = ctypes.cast(buf, P)
    assert fn(a, a, a, a, a, a, a, 16, 16, 16, 129, 128, None) == -1  # window beyond 128
    assert fn(None, a, a, a, a, a, a, 16, 16, 16, 128, 128, None) != 0
