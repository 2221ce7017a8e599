"""Full-size parity of the reference's own per-layer kernel sequence at
T >= 1040 (encoder.rs:1015-1081 FF2, :1104-1115 LayerNorm pair, :1471-1560
conv, :2099-2107 attention out), each kernel run at the sizes it serves and
compared with the CPU oracle on sampled rows of its GPU input:

* LayerNorm pair (encoder.cu:128-209), fp16 and fixed-scale e4m3 (x56)
  outputs: bit for bit;
* FF1 expand on that e4m3 at the fixed scale 8/448 with the packed x16 e4m3
  output (encoder.cu:1071-1077), then the FF contract at scale 1/16 with
  out += 0.5 Y (:1095-1103);
* FF2: LayerNorm -> dynamic INT4, s4 x s4 expand with SiLU -> x16 e4m3 and the
  2:4 compression (:1079-1085, epilogue 7), then the sparse contract on
  v_smfmac (:1087-1093) fed by that output -- at T = 45000 the contract's
  grid gives each workgroup several 256 x 256 tiles;
* conv pointwise 1 + GLU (:1121-1127) on the 256 x 256 engine's persistent
  tile loop, and conv pointwise 2 with out += Y (:1313-1319);
* attention out at scale 1/28 with out += Y (:2099-2107).

Tolerances: integer accumulators are exact, so the e4m3 codes of the SiLU
epilogues agree with the oracle except where the device exp moves an fp16
rounding boundary (>= 99 % of codes equal, the rest within one e4m3 step);
fp32-accumulated FP8 outputs within max|err| <= 1e-2 * RMS(output) (the
stated tolerance), and residual-updated outputs additionally with their
update (output - residual) within 2e-2 * RMS(update).
"""
import numpy as np
import pytest

from test_gpu_fullsize import assert_close, assert_fp8_close, host, note, rows_of, sample_rows

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

D, FF, CONV = 1024, 4096, 2048
FP8_INPUT_SCALE = 8.0 / 448.0  # encoder.rs:29


@pytest.fixture(scope="module")
def pk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import parakeet_linear

    return parakeet_linear


@pytest.fixture(scope="module")
def orc(oracle):
    oracle.set_threads(16)
    return oracle


def padded(t):
    return (t + 15) // 16 * 16


def fp16_weight(n, k, gen, scale=0.02):
    return (torch.randn((n, k), generator=gen, device="cuda") * scale).half()


def fp8_weight(pk, n, k, gen):
    """Request-time per-row FP8 weights (pk_quantize_rows, the generalised
    pk_quantize_rows1024 / _ffn_contract) from fp16 ~N(0, 0.02)."""
    w16 = fp16_weight(n, k, gen)
    q = torch.empty((n, k), dtype=torch.uint8, device="cuda")
    s = torch.empty(n, dtype=torch.float32, device="cuda")
    pk.call("pk_quantize_rows", 0, w16, q, s, n, n, k)
    return q, s


def check_residual(got, ref, before, what):
    """Stated form on the output, then the update alone."""
    assert_close(got, ref, what=what + " (output)")
    d_ref = ref.astype(np.float32) - before.astype(np.float32)
    d_got = got.astype(np.float32) - before.astype(np.float32)
    assert_close(d_got, d_ref, tol=2e-2, what=what + " (update)")


def ln_params(gen):
    g = (torch.rand(D, generator=gen, device="cuda") + 0.5).half()
    b = (torch.randn(D, generator=gen, device="cuda") * 0.1).half()
    return g, b


# ---- LayerNorm pair -------------------------------------------------------------------

@pytest.mark.parametrize("t,fp8", [(300, False), (300, True), (45000, False), (45000, True)])
def test_layer_norm_pair(pk, orc, t, fp8):
    pad = padded(t) + (16 if t % 16 == 0 else 0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1281 + t + int(fp8))
    x = (torch.randn((pad, D), generator=gen, device="cuda") * 2 + 0.3).half()
    g1, b1 = ln_params(gen)
    g2, b2 = ln_params(gen)
    out = torch.full((pad, D), 7.0, dtype=torch.float16, device="cuda")
    nxt = torch.full((pad, D), 0x55 if fp8 else 7, dtype=torch.uint8 if fp8 else torch.float16, device="cuda")
    inv = 448.0 / 8.0 if fp8 else 0.0
    note(f"layer_norm_pair T={t} padded={pad} fp8={fp8}")
    pk.call("pk_layer_norm_pair", x, g1, b1, out, g2, b2, nxt, t, pad, 1e-5, inv)
    idx = np.union1d(sample_rows(pad, 91 + int(fp8), per_strip=2), np.arange(t - 3, pad))
    r1, r2 = orc.layer_norm_pair(rows_of(x, idx), host(g1), host(b1), host(g2), host(b2), 1e-5, inv,
                                 valid_rows=int((idx < t).sum()))
    assert np.array_equal(rows_of(out, idx).view(np.uint16), r1.view(np.uint16))
    got2 = rows_of(nxt, idx)
    assert np.array_equal(got2.view(np.uint8 if fp8 else np.uint16), r2.view(np.uint8 if fp8 else np.uint16))


def test_layer_norm_pair_rejects(pk):
    x = torch.zeros((16, D), dtype=torch.float16, device="cuda")
    g = torch.ones(D, dtype=torch.float16, device="cuda")
    nxt = torch.zeros((16 * D + 8,), dtype=torch.uint8, device="cuda")
    with pytest.raises(pk.PkError):
        pk.call("pk_layer_norm_pair", x, g, g, x, g, g, nxt, 17, 16, 1e-5, 56.0)
    with pytest.raises(pk.PkError):  # e4m3 output must be 4-byte aligned
        pk.call("pk_layer_norm_pair", x, g, g, x, g, g, nxt[1:], 16, 16, 1e-5, 56.0)


# ---- FF1: fixed-scale FP8 expand (packed) -> FP8 contract -------------------------

@pytest.mark.parametrize("t", [7500, 45000])
def test_ff1_fixed_scale_chain(pk, orc, t):
    """LayerNorm pair (e4m3 x56) -> pk_ffn_expand_fp8_packed at scale 8/448
    -> pk_ffn_contract_fp8 (scale 1/16, out += 0.5 Y), each on 256-row tiles."""
    pad = padded(t)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1300 + t)
    x = (torch.randn((pad, D), generator=gen, device="cuda") * 2).half()
    g1, b1 = ln_params(gen)
    g2, b2 = ln_params(gen)
    state = torch.empty((pad, D), dtype=torch.float16, device="cuda")
    xq = torch.empty((pad, D), dtype=torch.uint8, device="cuda")
    pk.call("pk_layer_norm_pair", x, g1, b1, state, g2, b2, xq, t, pad, 1e-5, 1.0 / FP8_INPUT_SCALE)
    w1, s1 = fp8_weight(pk, FF, D, gen)
    w2, s2 = fp8_weight(pk, D, FF, gen)
    tile = pk.gemm_tile(pk.FMT_FP8, pk.EPI_F8, pad, FF)
    note(f"ffn_expand_fp8_packed T={t} tile={tile}")
    assert tile[0] == 256
    h = torch.empty((pad, FF), dtype=torch.uint8, device="cuda")
    pk.call("pk_ffn_expand_fp8_packed", xq, w1, s1, None, h, pad, FP8_INPUT_SCALE, 0)
    idx = sample_rows(pad, t + 1)
    acc = orc.gemm_e4m3(rows_of(xq, idx), host(w1))
    ref = orc.epilogue(acc, 1, host(s1), in_scale=FP8_INPUT_SCALE)
    assert_fp8_close(orc.e4m3_table(), rows_of(h, idx), ref, 0.99, f"expand_packed T={t}")
    tile = pk.gemm_tile(pk.FMT_FP8, pk.EPI_F16, pad, D)
    note(f"ffn_contract_fp8 T={t} tile={tile}")
    if t == 45000:
        assert tile[0] == 256
    before = rows_of(state, idx)
    pk.call("pk_ffn_contract_fp8", h, w2, s2, state, pad)
    ref = orc.epilogue(orc.gemm_e4m3(rows_of(h, idx), host(w2)), 2, host(s2), in_scale=1.0 / 16.0, residual=before)
    check_residual(rows_of(state, idx), ref, before, f"contract_fp8 T={t}")


# ---- FF2: LN -> INT4, s4 x s4 expand with 2:4 compression -> sparse contract ---------

@pytest.mark.parametrize("t", [7500, 45000])
def test_ff2_int4_sparse_chain(pk, orc, t):
    pad = padded(t)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1400 + t)
    x = (torch.randn((pad, D), generator=gen, device="cuda") * 2).half()
    g, b = ln_params(gen)
    xq = torch.empty((pad, D // 2), dtype=torch.uint8, device="cuda")
    xs = torch.empty(pad, dtype=torch.float32, device="cuda")
    pk.call("pk_layer_norm_quantize_int4_dynamic", x, g, b, xq, xs, t, pad, 1e-5)
    # FF2 expand weights: per-row INT4 (encoder.rs:367-407), packed on the GPU
    w16 = fp16_weight(FF, D, gen)
    wq = torch.empty((FF, D // 2), dtype=torch.uint8, device="cuda")
    ws = torch.empty(FF, dtype=torch.float32, device="cuda")
    pk.call("pk_pack_int4_rows", w16, FF, D, wq, ws)
    tile = pk.gemm_tile(pk.FMT_S4, pk.EPI_F8_24, pad, FF)
    note(f"ffn_expand_int4_sparse T={t} tile={tile}")
    assert tile[0] == 256
    buf = torch.empty(pad * (FF // 2 + FF // 8), dtype=torch.uint8, device="cuda")
    pk.call("pk_ffn_expand_int4_sparse", xq, wq, ws, xs, buf, pad, 1.0, 1)
    data = buf[: pad * FF // 2].view(pad, FF // 2)
    meta = buf[pad * FF // 2:].view(pad, FF // 8)
    idx = np.union1d(sample_rows(pad, t + 2), np.arange(t - 2, pad))
    acc = orc.gemm_s4(rows_of(xq, idx), host(wq)).astype(np.float32)
    dense = orc.epilogue(acc, 7, host(ws), row_scales=rows_of(xs, idx))
    rdata, rmeta = orc.compress_24(dense)
    gdata, gmeta = rows_of(data, idx), rows_of(meta, idx)
    assert np.mean(gdata == rdata) >= 0.99 and np.mean(gmeta == rmeta) >= 0.99, f"expand_int4_sparse T={t}"
    assert_fp8_close(orc.e4m3_table(), orc.decompress_24(gdata, gmeta), orc.decompress_24(rdata, rmeta), 0.99,
                     f"expand_int4_sparse T={t}")
    # padding rows (LN zero, INT4 zero, SiLU(0) = 0) compress to zero data
    assert not gdata[idx >= t].any()

    # the contract consumes that buffer as stored
    w2, s2 = fp8_weight(pk, D, FF, gen)
    state = torch.randn((pad, D), generator=gen, device="cuda").half()
    before = rows_of(state, idx)
    tiles = ((pad + 255) // 256) * (D // 256)
    note(f"ffn_contract_fp8_sparse T={t} tiles={tiles} (several per workgroup when > CUs)")
    pk.call("pk_ffn_contract_fp8_sparse", buf, w2, s2, state, pad, FF)
    acc = orc.gemm_e4m3(orc.decompress_24(gdata, gmeta), host(w2))
    ref = orc.epilogue(acc, 8, host(s2), in_scale=1.0 / 16.0, residual=before)
    check_residual(rows_of(state, idx), ref, before, f"contract_fp8_sparse T={t}")


# ---- conv: pointwise 1 + GLU, pointwise 2 + residual ---------------------------------

@pytest.mark.parametrize("t", [7500, 45000])
def test_conv_chain(pk, orc, t):
    pad = padded(t)
    valid = t
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1500 + t)
    x = torch.randn((pad, D), generator=gen, device="cuda").half()
    xq = torch.empty((pad, D), dtype=torch.uint8, device="cuda")
    xs = torch.empty(pad, dtype=torch.float32, device="cuda")
    pk.call("pk_quantize_rows1024", x, xq, xs, pad)
    w1, s1 = fp8_weight(pk, CONV, D, gen)
    out = torch.full((pad, D), 3.0, dtype=torch.float16, device="cuda")
    tile = pk.gemm_tile(pk.FMT_FP8, 6, pad, CONV)
    note(f"conv_glu_fp8 T={t} tile={tile} tiles={((pad + 255) // 256) * (CONV // 256)}")
    pk.call("pk_conv_glu_fp8", xq, w1, s1, xs, out, pad, valid)
    idx = np.union1d(sample_rows(pad, t + 3), np.arange(valid - 2, pad))
    ref = orc.epilogue(orc.gemm_e4m3(rows_of(xq, idx), host(w1)), 5, host(s1), row_scales=rows_of(xs, idx),
                       valid_rows=int((idx < valid).sum()))
    got = rows_of(out, idx)
    live = idx < valid
    assert not got[~live].astype(np.float32).any()
    assert_close(got[live], ref[live].astype(np.float32), what=f"conv_glu T={t}")

    # pointwise 2 on dynamic per-row FP8 of a fresh input, out += Y
    y = torch.randn((pad, D), generator=gen, device="cuda").half()
    yq = torch.empty((pad, D), dtype=torch.uint8, device="cuda")
    ys = torch.empty(pad, dtype=torch.float32, device="cuda")
    pk.call("pk_quantize_rows1024", y, yq, ys, pad)
    w2, s2 = fp8_weight(pk, D, D, gen)
    state = torch.randn((pad, D), generator=gen, device="cuda").half()
    before = rows_of(state, idx)
    note(f"conv_residual_fp8 T={t} tile={pk.gemm_tile(pk.FMT_FP8, pk.EPI_F16, pad, D)}")
    pk.call("pk_conv_residual_fp8", yq, w2, s2, ys, state, pad)
    ref = orc.epilogue(orc.gemm_e4m3(rows_of(yq, idx), host(w2)), 6, host(s2), row_scales=rows_of(ys, idx),
                       residual=before)
    check_residual(rows_of(state, idx), ref, before, f"conv_residual T={t}")


# ---- attention out ------------------------------------------------------------------

@pytest.mark.parametrize("t", [7500, 45000])
def test_attention_output(pk, orc, t):
    """o_proj on the e4m3 x28 attention context (pk_quantize_fp8_fixed at 28
    stands in for the attention kernel's output), out += Y."""
    pad = padded(t)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1600 + t)
    ctx = (torch.randn((pad, D), generator=gen, device="cuda") * 0.5).half()
    cq = torch.empty((pad, D), dtype=torch.uint8, device="cuda")
    pk.call("pk_quantize_fp8_fixed", ctx, cq, pad * D, 28.0)
    w, s = fp8_weight(pk, D, D, gen)
    state = torch.randn((pad, D), generator=gen, device="cuda").half()
    idx = sample_rows(pad, t + 4)
    before = rows_of(state, idx)
    note(f"attention_output_fp8 T={t} tile={pk.gemm_tile(pk.FMT_FP8, pk.EPI_F16, pad, D)}")
    pk.call("pk_attention_output_fp8", cq, w, s, state, pad)
    ref = orc.epilogue(orc.gemm_e4m3(rows_of(cq, idx), host(w)), 6, host(s), in_scale=1.0 / 28.0, residual=before)
    check_residual(rows_of(state, idx), ref, before, f"attention_output T={t}")


# ---- FF2 on the operand form of the INT4 codes ---------------------------------------

def nibbles_to_codes(packed):
    """byte j = q[2j] & 15 | q[2j+1] << 4 -> signed codes in k order (closed form)."""
    p = packed.astype(np.int16)
    lo, hi = p & 15, p >> 4
    codes = np.stack([lo, hi], axis=-1).reshape(packed.shape[0], -1)
    return np.where(codes >= 8, codes - 16, codes).astype(np.int8)


@pytest.mark.parametrize("t", [7500, 45000])
def test_ff2_int4_codes_equal_packed(pk, orc, t):
    """pk_layer_norm_quantize_int4_codes writes the codes of the packed
    producer (same scales), pk_unpack_int4 is the closed-form sign extension,
    and pk_ffn_expand_int4_sparse_codes on the codes writes exactly the bytes
    pk_ffn_expand_int4_sparse writes on the nibble pairs (same int32
    accumulators, same epilogue)."""
    pad = padded(t) + 16
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1700 + t)
    x = (torch.randn((pad, D), generator=gen, device="cuda") * 2).half()
    g, b = ln_params(gen)
    xq = torch.empty((pad, D // 2), dtype=torch.uint8, device="cuda")
    xs = torch.empty(pad, dtype=torch.float32, device="cuda")
    xc = torch.full((pad, D), 5, dtype=torch.int8, device="cuda")
    xcs = torch.empty(pad, dtype=torch.float32, device="cuda")
    note(f"int4 codes producer T={t} padded={pad}")
    pk.call("pk_layer_norm_quantize_int4_dynamic", x, g, b, xq, xs, t, pad, 1e-5)
    pk.call("pk_layer_norm_quantize_int4_codes", x, g, b, xc, xcs, t, pad, 1e-5)
    assert torch.equal(xs, xcs)
    idx = np.union1d(sample_rows(pad, t + 5, per_strip=2), np.arange(t - 2, pad))
    assert np.array_equal(rows_of(xc, idx), nibbles_to_codes(rows_of(xq, idx)))
    xu = torch.empty((pad, D), dtype=torch.int8, device="cuda")
    pk.call("pk_unpack_int4", xq, xu, pad * D)
    assert torch.equal(xu, xc)
    w16 = fp16_weight(FF, D, gen)
    wq = torch.empty((FF, D // 2), dtype=torch.uint8, device="cuda")
    ws = torch.empty(FF, dtype=torch.float32, device="cuda")
    pk.call("pk_pack_int4_rows", w16, FF, D, wq, ws)
    wc = torch.empty((FF, D), dtype=torch.int8, device="cuda")
    pk.call("pk_unpack_int4", wq, wc, FF * D)
    assert np.array_equal(host(wc), nibbles_to_codes(host(wq)))
    a = torch.empty(pad * (FF // 2 + FF // 8), dtype=torch.uint8, device="cuda")
    c = torch.full_like(a, 0x33)
    note(f"ffn_expand_int4_sparse_codes T={t} tile={pk.gemm_tile(pk.FMT_I8, pk.EPI_F8_24, pad, FF)}")
    pk.call("pk_ffn_expand_int4_sparse", xq, wq, ws, xs, a, pad, 1.0, 1)
    pk.call("pk_ffn_expand_int4_sparse_codes", xc, wc, ws, xs, c, pad, 1.0, 1)
    assert torch.equal(a, c)
