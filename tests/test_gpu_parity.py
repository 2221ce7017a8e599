"""GPU parity: every HIP entry point against the CPU oracle on seeded inputs.

Integer, byte and index results are compared bit-exactly; fp32-accumulated
FP8 / FP16 / INT4-g128 outputs within max|err| <= 1e-2 * RMS(reference output),
the tolerance BASELINE.json's north star states.  All calls go through the
C ABI (parakeet_linear is a ctypes mirror of include/pk_linear.h).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 1e-2


@pytest.fixture(scope="module")
def pk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import parakeet_linear

    return parakeet_linear


@pytest.fixture(scope="module")
def orc(oracle):
    oracle.set_threads(8)
    return oracle


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(t, dtype=None):
    torch.cuda.synchronize()
    a = t.cpu()
    if a.dtype == torch.float16:
        return a.view(torch.int16).numpy().view(np.float16)
    return a.numpy() if dtype is None else a.numpy().view(dtype)


def empty(shape, dtype):
    return torch.empty(shape, dtype=dtype, device="cuda")


def note(msg):
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


def assert_close(got, ref, tol=TOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    err = np.max(np.abs(got - ref))
    assert np.isfinite(got).all()
    assert err <= tol * rms, f"max err {err} > {tol} * rms {rms}"


def assert_fp8_close(table, got, ref, exact_frac=0.99):
    """Requantized e4m3 outputs of an fp32-accumulated GEMM: codes agree almost
    everywhere; where the summation order moved a rounding boundary they differ
    by at most one e4m3 step (relative 2^-3, or the 2^-9 subnormal step)."""
    assert np.mean(got == ref) >= exact_frac
    g, r = table[got].astype(np.float64), table[ref].astype(np.float64)
    assert np.all(np.abs(g - r) <= np.abs(r) / 8 + 2.0 ** -9 + 1e-12)


def weights(n, k, seed, sigma=0.02):
    return (np.random.default_rng(seed).standard_normal((n, k)) * sigma).astype(np.float16)


def acts(m, k, seed, outliers=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if outliers:
        mask = rng.random((m, k)) < 1e-3
        x[mask] = np.where(rng.random(mask.sum()) < 0.5, -20.0, 20.0)
    return x.astype(np.float16)


# ---- conversions and quantizers (bit-exact) ---------------------------------------

def test_quantize_fp8_all_fp16_inputs(pk, orc):
    note("quantize_fp8 exhaustive")
    allh = np.arange(65536, dtype=np.uint16).view(np.float16)
    allh = allh[np.isfinite(allh.astype(np.float32))]
    x = dev(allh)
    out = empty(allh.size, torch.uint8)
    for inv in (1.0, 56.0, 448.0 / 0.125, 1.0 / 3.0, 3.7e-3):
        pk.launch_fp8_quantize(x, out, inv)
        assert np.array_equal(host(out), orc.quantize_fp8_static(allh, inv)), inv


def test_quantize_int8_all_fp16_inputs(pk, orc):
    note("quantize_int8 exhaustive")
    allh = np.arange(65536, dtype=np.uint16).view(np.float16)
    allh = allh[np.isfinite(allh.astype(np.float32))]
    x = dev(allh)
    out = empty(allh.size, torch.int8)
    for inv in (1.0, 127.0 / 0.125, 0.37):
        pk.launch_int8_quantize(x, out, inv)
        assert np.array_equal(host(out), orc.quantize_int8_static(allh, inv)), inv


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("m,k,valid", [(1, 1024, 1), (37, 1024, 30), (16, 4096, 16), (5, 256, 5), (3, 8, 3),
                                        (9, 1032, 7), (6, 8192, 5), (4, 6152, 4)])
def test_quantize_rows(pk, orc, kind, m, k, valid):
    note(f"quantize_rows kind={kind} m={m} k={k}")
    x = acts(m, k, 100 + m + k)
    if m > 2:
        x[1] = 0  # all-zero row -> scale 1
    out = empty((m, k // 2 if kind == 2 else k), torch.uint8)
    scales = empty(m, torch.float32)
    pk.call("pk_quantize_rows", kind, dev(x), out, scales, m, valid, k)
    ref = {0: orc.quantize_fp8_rows, 1: orc.quantize_int8_rows, 2: orc.quantize_int4_rows}[kind](x, valid)
    assert np.array_equal(host(out).view(np.uint8), ref[0].view(np.uint8))
    assert np.array_equal(host(scales), ref[1])


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("k", [1024, 4096])
def test_quantize_rows_all_fp16_inputs(pk, orc, kind, k):
    """Every finite fp16 x with |x| <= M goes through x / scale for twelve row
    maxima M (each row holds M, -M and a run of the enumeration): the kernel's
    quotient must round exactly as the oracle's IEEE division does, ties and
    near-ties at the rounding boundaries included."""
    note(f"quantize_rows exhaustive kind={kind} k={k}")
    allh = np.arange(65536, dtype=np.uint16).view(np.float16)
    allh = allh[np.isfinite(allh.astype(np.float32))]
    rows = []
    for mx in (65504.0, 448.0, 127.0, 100.0, 37.3, 7.0, 1.0, 0.3, 1.0 / 3.0, 6.1e-5, 1e-6, 6e-8):
        m = np.float16(mx)
        vals = allh[np.abs(allh.astype(np.float32)) <= np.float32(m)]
        per = k - 2
        for i in range(0, vals.size, per):
            r = np.zeros(k, np.float16)
            r[0], r[1] = m, -m
            chunk = vals[i:i + per]
            r[2:2 + chunk.size] = chunk
            rows.append(r)
    x = np.stack(rows)
    m = x.shape[0]
    out = empty((m, k // 2 if kind == 2 else k), torch.uint8)
    scales = empty(m, torch.float32)
    pk.call("pk_quantize_rows", kind, dev(x), out, scales, m, m, k)
    ref = {0: orc.quantize_fp8_rows, 1: orc.quantize_int8_rows, 2: orc.quantize_int4_rows}[kind](x, m)
    assert np.array_equal(host(scales), ref[1])
    assert np.array_equal(host(out).view(np.uint8), ref[0].view(np.uint8))


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("k", [1024, 4096])
def test_quantize_rows_non_finite(pk, orc, kind, k):
    """Rows holding inf, -inf or NaN next to ordinary values, and rows of
    ordinary values only, in one launch (the kernel picks a path per row)."""
    note(f"quantize_rows non-finite kind={kind} k={k}")
    x = acts(12, k, 77 + k)
    x[1, 5] = np.inf
    x[3, 0] = -np.inf
    x[5, 9] = np.nan
    x[7, 1:4] = [np.nan, np.inf, -np.inf]
    x[9] = np.nan
    out = empty((12, k // 2 if kind == 2 else k), torch.uint8)
    scales = empty(12, torch.float32)
    pk.call("pk_quantize_rows", kind, dev(x), out, scales, 12, 12, k)
    ref = {0: orc.quantize_fp8_rows, 1: orc.quantize_int8_rows, 2: orc.quantize_int4_rows}[kind](x, 12)
    assert np.array_equal(host(scales), ref[1], equal_nan=True)
    assert np.array_equal(host(out).view(np.uint8), ref[0].view(np.uint8))


@pytest.mark.parametrize("int4", [False, True])
def test_layer_norm_quantize_non_finite(pk, orc, int4):
    """Rows with inf / NaN inputs, a row whose fp16 output overflows (gamma
    large), and ordinary rows: each row's path must match the oracle."""
    note(f"layer_norm_quantize non-finite int4={int4}")
    m = 8
    x = (acts(m, 1024, 17).astype(np.float32) * 2).astype(np.float16)
    x[1, 3] = np.inf
    x[2, 7] = np.nan
    x[4] = 0  # constant row: variance 0
    x[5, 0] = 3000.0  # one large outlier: normalized value near sqrt(1023)
    g = np.random.default_rng(18).uniform(0.5, 1.5, 1024).astype(np.float16)
    g[0] = 30000.0  # feature 0 overflows fp16 in row 5
    b = (np.random.default_rng(19).standard_normal(1024) * 0.1).astype(np.float16)
    out = empty((m, 512 if int4 else 1024), torch.uint8)
    scales = empty(m, torch.float32)
    name = "pk_layer_norm_quantize_int4_dynamic" if int4 else "pk_layer_norm_quantize_fp8_dynamic"
    pk.call(name, dev(x), dev(g), dev(b), out, scales, m, m, 1e-5)
    q, s, _ = orc.layer_norm_quantize(x, g, b, 1e-5, int4, valid_rows=m)
    assert np.array_equal(host(scales), s, equal_nan=True)
    assert np.array_equal(host(out), q)


@pytest.mark.parametrize("int4", [False, True])
def test_layer_norm_quantize(pk, orc, int4):
    note(f"layer_norm_quantize int4={int4}")
    m, pad = 45, 48
    x = (acts(pad, 1024, 7).astype(np.float32) * 2 + 0.5).astype(np.float16)
    g = np.random.default_rng(8).uniform(0.5, 1.5, 1024).astype(np.float16)
    b = (np.random.default_rng(9).standard_normal(1024) * 0.1).astype(np.float16)
    out = empty((pad, 512 if int4 else 1024), torch.uint8)
    scales = empty(pad, torch.float32)
    name = "pk_layer_norm_quantize_int4_dynamic" if int4 else "pk_layer_norm_quantize_fp8_dynamic"
    pk.call(name, dev(x), dev(g), dev(b), out, scales, m, pad, 1e-5)
    q, s, _ = orc.layer_norm_quantize(x, g, b, 1e-5, int4, valid_rows=m)
    assert np.array_equal(host(scales), s)
    assert np.array_equal(host(out), q)


@pytest.mark.parametrize("kind", ["fp8", "int8", "int4"])
def test_pack_rows(pk, orc, kind):
    note(f"pack_rows {kind}")
    n, k = 300, 1024
    w = weights(n, k, 11)
    w[5] = 0
    width = k // 2 if kind == "int4" else k
    q = empty((n, width), torch.uint8)
    s = empty(n, torch.float32)
    pk.call(f"pk_pack_{kind}_rows", dev(w), n, k, q, s)
    rq, rs = {"fp8": orc.pack_fp8_rows, "int8": orc.pack_int8_rows, "int4": orc.pack_int4_rows}[kind](w)
    assert np.array_equal(host(q).view(np.uint8), rq.view(np.uint8))
    assert np.array_equal(host(s), rs)


def test_pack_int4_g128(pk, orc):
    note("pack_int4_g128")
    n, k = 200, 1024
    w = weights(n, k, 12)
    w[3, 128:256] = 0
    q = empty((n, k // 8), torch.int32)
    s = empty((n, k // 128), torch.float16)
    z = empty((n, k // 128), torch.float16)
    pk.call("pk_pack_int4_g128", dev(w), n, k, q, s, z)
    rq, rs, rz = orc.pack_int4_g128(w)
    assert np.array_equal(host(q).view(np.uint32), rq)
    assert np.array_equal(host(s).view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(host(z).view(np.uint16), rz.view(np.uint16))


# ---- INT8 x INT8 -> INT32 (bit-exact) ------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(750, 4096, 1024), (1, 640, 1024), (257, 1040, 4096), (17, 16, 128)])
def test_int8_accumulators_exact(pk, orc, m, n, k):
    note(f"int8 accumulate m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 7 + n)
    x = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    acc = empty((m, n), torch.int32)
    pk.call("pk_linear_int8_accumulate", dev(x), dev(w), acc, m, n, k)
    assert np.array_equal(host(acc), orc.gemm_i8(x, w))


def test_int8_linear_epilogue_config1(pk, orc):
    """W[4096x1024] ~N(0,0.02) -> per-row INT8, x[750x1024]."""
    note("int8 linear config 1")
    m, n, k = 750, 4096, 1024
    w = weights(n, k, 0x5EED0001)
    x = acts(m, k, 0x5EED0002, outliers=False)
    wq, ws = orc.pack_int8_rows(w)
    in_scale = 0.125 / 127.0 * 32  # covers |x| <= ~4
    xq = orc.quantize_int8_static(x, 1.0 / in_scale)
    bias = (np.random.default_rng(3).standard_normal(n) * 0.1).astype(np.float32)
    out = empty((m, n), torch.float16)
    pk.launch_int8_linear(dev(xq), dev(wq), dev(ws), dev(bias), out, m, n, k, in_scale, 0)
    ref = orc.epilogue_quantized(orc.gemm_i8(xq, wq).astype(np.float32), in_scale, ws, bias, 0)
    assert np.array_equal(host(out).view(np.uint16), ref.view(np.uint16))
    pk.launch_int8_linear(dev(xq), dev(wq), dev(ws), dev(bias), out, m, n, k, in_scale, 1)
    ref = orc.epilogue_quantized(orc.gemm_i8(xq, wq).astype(np.float32), in_scale, ws, bias, 1)
    assert_close(host(out), ref.astype(np.float32))


def test_int8_dynamic_exact(pk, orc):
    note("int8 dyn")
    m, n, k = 300, 1024, 4096
    x = acts(m, k, 21)
    w = weights(n, k, 22)
    xq, xs = orc.quantize_int8_rows(x)
    wq, ws = orc.pack_int8_rows(w)
    out = empty((m, n), torch.float32)
    pk.call("pk_linear_int8_dyn", dev(xq), dev(xs), dev(wq), dev(ws), None, out, 1, m, n, k)
    acc = orc.gemm_i8(xq, wq).astype(np.float32)
    ref = (acc * xs[:, None]).astype(np.float32) * ws[None, :]
    assert np.array_equal(host(out), ref.astype(np.float32))


# ---- s4 x s4 -------------------------------------------------------------------------

def test_int4_accumulators_exact(pk, orc):
    note("int4 accumulate")
    m, n, k = 301, 512, 1024
    rng = np.random.default_rng(31)
    x = rng.integers(0, 256, (m, k // 2), dtype=np.uint8)
    w = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    acc = empty((m, n), torch.int32)
    pk.call("pk_linear_int4_accumulate", dev(x), dev(w), acc, m, n, k)
    assert np.array_equal(host(acc), orc.gemm_s4(x, w))


def test_ffn_expand_int4_sparse(pk, orc):
    note("ffn_expand_int4_sparse")
    rows = 300
    x = acts(rows, 1024, 41)
    w = weights(4096, 1024, 42)
    xq, xs = orc.quantize_int4_rows(x)
    wq, ws = orc.pack_int4_rows(w)
    out = empty(rows * 2048 + rows * 512, torch.uint8)
    pk.call("pk_ffn_expand_int4_sparse", dev(xq), dev(wq), dev(ws), dev(xs), out, rows, 1.0, 1)
    got = host(out)
    data, meta = got[: rows * 2048].reshape(rows, 2048), got[rows * 2048:].reshape(rows, 512)
    acc = orc.gemm_s4(xq, wq).astype(np.float32)
    dense = orc.epilogue(acc, 7, ws, row_scales=xs)
    rdata, rmeta = orc.compress_24(dense)
    # exact int32 accumulators; only SiLU's exp may differ by an ulp, which can
    # move an fp16 rounding boundary, so compare codes almost everywhere and the
    # decompressed values within one fp8 step
    assert np.mean(data == rdata) > 0.999 and np.mean(meta == rmeta) > 0.999
    assert_fp8_close(orc.e4m3_table(), orc.decompress_24(data, meta), orc.decompress_24(rdata, rmeta), 0.999)


# ---- FP8 -------------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(750, 4096, 1024), (33, 1024, 4096), (1, 3072, 1024)])
def test_fp8_linear_epilogue(pk, orc, m, n, k):
    note(f"fp8 linear m={m} n={n} k={k}")
    w = weights(n, k, 51)
    x = acts(m, k, 52)
    wq, ws = orc.pack_fp8_rows(w)
    in_scale = 8.0 / 448.0
    xq = orc.quantize_fp8_static(x, 1.0 / in_scale)
    bias = (np.random.default_rng(53).standard_normal(n) * 0.05).astype(np.float32)
    out = empty((m, n), torch.float16)
    pk.launch_fp8_linear(dev(xq), dev(wq), dev(ws), dev(bias), out, m, n, k, in_scale, 0)
    ref = orc.epilogue_quantized(orc.gemm_e4m3(xq, wq), in_scale, ws, bias, 0)
    assert_close(host(out), ref.astype(np.float32))


def test_fp8_dynamic_fp32_out(pk, orc):
    note("fp8 dyn fp32")
    m, n, k = 515, 2048, 1024
    x = acts(m, k, 61)
    w = weights(n, k, 62)
    xq, xs = orc.quantize_fp8_rows(x)
    wq, ws = orc.pack_fp8_rows(w)
    out = empty((m, n), torch.float32)
    pk.call("pk_linear_fp8_dyn", dev(xq), dev(xs), dev(wq), dev(ws), None, out, 1, m, n, k)
    ref = orc.gemm_e4m3(xq, wq) * xs[:, None] * ws[None, :]
    assert_close(host(out), ref)


def test_ffn_expand_fp8_and_packed(pk, orc):
    note("ffn_expand_fp8 (+packed)")
    rows = 260
    x = acts(rows, 1024, 71)
    w = weights(4096, 1024, 72)
    wq, ws = orc.pack_fp8_rows(w)
    in_scale = 8.0 / 448.0
    xq = orc.quantize_fp8_static(x, 1.0 / in_scale)
    acc = orc.gemm_e4m3(xq, wq)
    out = empty((rows, 4096), torch.float16)
    pk.call("pk_ffn_expand_fp8", dev(xq), dev(wq), dev(ws), None, out, rows, in_scale, 0)
    assert_close(host(out), orc.epilogue(acc, 0, ws, in_scale=in_scale).astype(np.float32))
    packed = empty((rows, 4096), torch.uint8)
    pk.call("pk_ffn_expand_fp8_packed", dev(xq), dev(wq), dev(ws), None, packed, rows, in_scale, 0)
    ref = orc.epilogue(acc, 1, ws, in_scale=in_scale)
    assert_fp8_close(orc.e4m3_table(), host(packed), ref)


@pytest.mark.parametrize("name", ["pk_ffn_contract_fp8", "pk_conv_residual_fp8", "pk_attention_output_fp8"])
def test_residual_linears(pk, orc, name):
    note(name)
    rows = 300
    k = 4096 if name == "pk_ffn_contract_fp8" else 1024
    x = acts(rows, k, 81)
    w = weights(1024, k, 82)
    wq, ws = orc.pack_fp8_rows(w)
    residual = acts(rows, 1024, 83, outliers=False)
    out = dev(residual.copy())
    if name == "pk_conv_residual_fp8":
        xq, xs = orc.quantize_fp8_rows(x)
        pk.call(name, dev(xq), dev(wq), dev(ws), dev(xs), out, rows)
        ref = orc.epilogue(orc.gemm_e4m3(xq, wq), 6, ws, row_scales=xs, residual=residual)
    else:
        in_scale = 1.0 / 16.0 if name == "pk_ffn_contract_fp8" else 1.0 / 28.0
        xq = orc.quantize_fp8_static(x, 1.0 / in_scale)
        pk.call(name, dev(xq), dev(wq), dev(ws), out, rows)
        mode = 2 if name == "pk_ffn_contract_fp8" else 6
        ref = orc.epilogue(orc.gemm_e4m3(xq, wq), mode, ws, in_scale=in_scale, residual=residual)
    assert_close(host(out).astype(np.float32), ref.astype(np.float32))  # 1e-2 * RMS(output)
    delta_ref = ref.astype(np.float32) - residual.astype(np.float32)
    delta_got = host(out).astype(np.float32) - residual.astype(np.float32)
    assert_close(delta_got, delta_ref, tol=2e-2)  # the update alone


# ---- FP16 ------------------------------------------------------------------------------

@pytest.mark.parametrize("act", [0, 1, 2])
def test_fp16_linear_epilogue(pk, orc, act):
    note(f"fp16 linear act={act}")
    m, n, k = 200, 640, 1024
    x = acts(m, k, 91, outliers=False)
    w = weights(n, k, 92)
    bias = (np.random.default_rng(93).standard_normal(n) * 0.1).astype(np.float32)
    res = acts(m, n, 94, outliers=False)
    out = empty((m, n), torch.float16)
    pk.launch_linear(dev(x), dev(w), dev(bias), dev(res), out, m, n, k, 0.5, 0.25, act)
    ref = orc.epilogue_linear(orc.gemm_f16(x, w), bias, res, 0.5, 0.25, act)
    assert_close(host(out), ref.astype(np.float32))


def test_fp16_qkv(pk, orc):
    note("fp16 qkv")
    m, n, k = 130, 1024, 1024
    x = acts(m, k, 95, outliers=False)
    ws = [weights(n, k, 96 + i) for i in range(3)]
    out = empty((3, m, n), torch.float16)
    pk.call("pk_linear_fp16_qkv", dev(x), dev(ws[0]), dev(ws[1]), dev(ws[2]), out, m, n, k)
    got = host(out)
    for i in range(3):
        assert_close(got[i], orc.gemm_f16(x, ws[i]))


# ---- INT4 g128 ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(750, 4096, 1024), (97, 1024, 4096)])
def test_int4g128_a16(pk, orc, m, n, k):
    note(f"g128 a16 m={m} n={n} k={k}")
    x = acts(m, k, 101, outliers=False)
    w = weights(n, k, 102)
    q, s, z = orc.pack_int4_g128(w)
    out = empty((m, n), torch.float32)
    pk.call("pk_linear_int4g128", dev(x), dev(q), dev(s), dev(z), None, out, 1, m, n, k)
    assert_close(host(out), orc.gemm_g128_a16(x, q, s, z))


@pytest.mark.parametrize("m,n,k", [(750, 4096, 1024), (97, 1024, 4096), (300, 1040, 1024)])
def test_int4g128_a8_exact(pk, orc, m, n, k):
    """INT4-g128 weights x INT8 activations: fp32 outputs bit-exact against
    the oracle (the last case's ragged column tile reads clamped weight rows
    through the same XOR-keyed LDS layout)."""
    note(f"g128 a8 m={m} n={n} k={k}")
    x = acts(m, k, 111)
    w = weights(n, k, 112)
    q, s, z = orc.pack_int4_g128(w)
    xq, xs = orc.quantize_int8_rows(x)
    out = empty((m, n), torch.float32)
    pk.call("pk_linear_int4g128_a8", dev(xq), dev(xs), dev(q), dev(s), dev(z), None, out, 1, m, n, k)
    parts = pk.gemm_k_split(pk.FMT_G128A8, pk.EPI_F32, m, n, k)
    ref = orc.gemm_g128_a8(xq, xs, q, s, z, parts=parts)
    assert np.array_equal(host(out), ref), f"K split {parts}"


# ---- Q4_K ----------------------------------------------------------------------------------

def q4k_random_blocks(n, k, seed):
    """Raw Q4_K blocks with arbitrary scale/min/quant bytes and finite d, dmin."""
    rng = np.random.default_rng(seed)
    blocks = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    d = (rng.random((n, k // 256, 2)) * 2e-3).astype(np.float16)
    blocks[..., 0:4] = d.view(np.uint8).reshape(n, k // 256, 4)
    return blocks


@pytest.mark.parametrize("source", ["encoded", "random"])
def test_q4k_dequantize_exact(pk, orc, source):
    n, k = 40, 1024
    note(f"q4k dequantize {source} n={n} k={k}")
    blocks = orc.q4k_encode(weights(n, k, 130)) if source == "encoded" else q4k_random_blocks(n, k, 131)
    out = empty((n, k), torch.float16)
    pk.call("pk_q4_k_dequantize", dev(blocks), out, n, k)
    ref = orc.q4k_dequant(blocks).astype(np.float16)
    assert np.array_equal(host(out).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("m,n,k,act", [(300, 272, 512, 0), (97, 1024, 1024, 2), (130, 256, 768, 1)])
def test_q4k_linear_epilogue(pk, orc, m, n, k, act):
    note(f"q4k linear m={m} n={n} k={k} act={act}")
    x = acts(m, k, 132, outliers=False)
    blocks = orc.q4k_encode(weights(n, k, 133))
    bias = (np.random.default_rng(134).standard_normal(n) * 0.1).astype(np.float32)
    out = empty((m, n), torch.float16)
    pk.call("pk_q4_k_linear_epilogue", dev(x), dev(blocks), dev(bias), out, m, n, k, act)
    ref = orc.epilogue_linear(orc.gemm_q4k(x, blocks), bias=bias, activation=act)
    assert_close(host(out), ref)


def test_q4k_linear_multi_tile(pk):
    """More 256x256 tiles than workgroups (each runs several): fp16 output of
    the fused kernel against the device dequantization (pinned bit-exact
    above) followed by an fp32 torch matmul."""
    m, n, k = 10240, 2048, 512
    note(f"q4k linear multi-tile m={m} n={n} k={k}")
    gen = torch.Generator(device="cuda").manual_seed(135)
    x = torch.randn((m, k), device="cuda", generator=gen).half()
    blocks = torch.from_numpy(q4k_random_blocks(n, k, 136)).cuda()
    deq = empty((n, k), torch.float16)
    pk.call("pk_q4_k_dequantize", blocks, deq, n, k)
    out = empty((m, n), torch.float16)
    pk.call("pk_q4_k_linear_epilogue", x, blocks, None, out, m, n, k, 0)
    torch.backends.cuda.matmul.allow_tf32 = False
    ref = (x.float() @ deq.float().t()).half().float()
    assert_close(host(out).astype(np.float32), ref.cpu().numpy())


@pytest.mark.parametrize("fmt", ["g128a16", "g128a8"])
def test_g128_staged_fp16_multi_tile(pk, orc, fmt):
    """fp16 outputs leave through the LDS staging area while the next tile's
    first K-step loads; with more tiles than workgroups they must equal the
    fp32 outputs (register epilogue) rounded to fp16, bit for bit."""
    m, n, k = 10240, 2048, 512
    note(f"g128 staged fp16 {fmt} m={m} n={n} k={k}")
    w = weights(n, k, 137)
    q, s, z = orc.pack_int4_g128(w)
    rng = np.random.default_rng(138)
    if fmt == "g128a16":
        a = dev(acts(m, k, 139, outliers=False))
        f, rs = pk.FMT_G128A16, None
    else:
        a = torch.from_numpy(rng.integers(-127, 128, (m, k), dtype=np.int8)).cuda()
        f, rs = pk.FMT_G128A8, dev((rng.random(m) * 1e-2 + 1e-3).astype(np.float32))
    o16 = empty((m, n), torch.float16)
    o32 = empty((m, n), torch.float32)
    for epi, o in ((pk.EPI_F16, o16), (pk.EPI_F32, o32)):
        pk.gemm(f, epi, a, dev(q), m, n, k, o, row_scales=rs, g_scales=dev(s), g_zeros=dev(z))
    assert np.array_equal(host(o16).view(np.uint16), host(o32).astype(np.float16).view(np.uint16))


# ---- joint ---------------------------------------------------------------------------------

@pytest.mark.parametrize("int8", [False, True])
def test_joint_gemv(pk, orc, int8):
    note(f"joint int8={int8}")
    outputs, hidden, steps = 1030, 640, 7
    rng = np.random.default_rng(120)
    w16 = (rng.standard_normal((outputs, hidden)) * 0.05).astype(np.float16)
    bias = (rng.standard_normal(outputs) * 0.1).astype(np.float32)
    enc = rng.standard_normal((steps, hidden)).astype(np.float16)
    pred = rng.standard_normal(hidden).astype(np.float32)
    scores = empty((steps, outputs), torch.float32)
    decision = empty((steps, 2), torch.int32)
    if int8:
        wq, ws = orc.pack_int8_rows(w16)
        pk.call("pk_joint_gemv", dev(wq), 1, dev(ws), dev(bias), dev(enc), dev(pred), scores, decision,
                outputs, hidden, 1025, 5, steps, hidden)
    else:
        pk.call("pk_joint_gemv", dev(w16), 0, None, dev(bias), dev(enc), dev(pred), scores, decision,
                outputs, hidden, 1025, 5, steps, hidden)
    got = host(scores)
    dec = host(decision)
    for t in range(steps):
        if int8:
            ref = orc.joint_scores_i8(wq, ws, bias, enc[t], pred)
        else:
            ref = orc.joint_scores_f16(w16, bias, enc[t], pred)
        assert_close(got[t], ref, tol=1e-4)
        assert tuple(dec[t]) == orc.joint_decide(got[t])


# ---- conv GLU and subsampling linears ---------------------------------------------

def test_conv_glu_fp8(pk, orc):
    note("conv_glu_fp8")
    rows, valid = 300, 290
    x = acts(rows, 1024, 131)
    w = weights(2048, 1024, 132)
    xq, xs = orc.quantize_fp8_rows(x)
    wq, ws = orc.pack_fp8_rows(w)
    out = empty((rows, 1024), torch.float16)
    pk.call("pk_conv_glu_fp8", dev(xq), dev(wq), dev(ws), dev(xs), out, rows, valid)
    ref = orc.epilogue(orc.gemm_e4m3(xq, wq), 5, ws, row_scales=xs, valid_rows=valid)
    got = host(out)
    assert not got[valid:].astype(np.float32).any()
    assert_close(got[:valid], ref[:valid].astype(np.float32))


@pytest.mark.parametrize("name,n,k,mode", [("pk_subsample_projection_fp8", 1024, 4096, 3),
                                           ("pk_subsample_pointwise_fp8", 256, 256, 4)])
def test_subsample_linears(pk, orc, name, n, k, mode):
    note(name)
    rows = 333
    x = acts(rows, k, 141)
    w = weights(n, k, 142)
    bias = (np.random.default_rng(143).standard_normal(n) * 0.1).astype(np.float32)
    xq, xs = orc.quantize_fp8_rows(x)
    wq, ws = orc.pack_fp8_rows(w)
    out = empty((rows, n), torch.float16)
    pk.call(name, dev(xq), dev(wq), dev(ws), dev(xs), dev(bias), out, rows)
    ref = orc.epilogue(orc.gemm_e4m3(xq, wq), mode, ws, row_scales=xs, bias=bias)
    assert_close(host(out), ref.astype(np.float32))


# ---- activation-sparse FF2 (INT8, row skip) -------------------------------------

def sparse_acts(rows, k, keep, seed, dead_blocks=0):
    """SiLU-like fp16 activations keeping each frame's top `keep` fraction of
    magnitudes (the rest exactly 0); the last `dead_blocks` 16-row blocks are all
    zero (padding frames), which the kernel must skip."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x = x / (1 + np.exp(-x))
    kth = int(round(k * (1 - keep)))
    thresh = np.partition(np.abs(x), kth, axis=1)[:, kth:kth + 1]
    x[np.abs(x) < thresh] = 0
    if dead_blocks:
        x[rows - 16 * dead_blocks:] = 0
    return x.astype(np.float16)


@pytest.mark.parametrize("sparsity", [0.5, 0.8, 0.9, 0.95])
def test_ffn_contract_int8_rowskip_exact(pk, orc, sparsity):
    note(f"int8 rowskip sparsity={sparsity}")
    rows = 512
    x = sparse_acts(rows, 4096, 1 - sparsity, 151, dead_blocks=3)
    w = weights(1024, 4096, 152)
    xq, xs = orc.quantize_int8_rows(x)
    wq, ws = orc.pack_int8_rows(w)
    out = empty((rows, 1024), torch.float32)
    counts = torch.zeros(2, dtype=torch.int32, device="cuda")
    pk.call("pk_ffn_contract_int8_rowskip", dev(xq), dev(xs), dev(wq), dev(ws), out, rows, counts)
    acc = orc.gemm_i8(xq, wq).astype(np.float32)
    ref = (acc * xs[:, None]).astype(np.float32) * ws[None, :]
    assert np.array_equal(host(out), ref.astype(np.float32))
    skipped, total = (int(v) for v in host(counts))
    tiles = ((rows + 255) // 256) * (1024 // 256)
    assert total == tiles * 8 * 8 * (4096 // 128)  # tiles x waves x row blocks x K-steps
    # the three dead 16-row blocks, every K-step, seen by the 4 column waves of each of 4 column tiles
    assert skipped >= 3 * 32 * 4 * 4


# ---- 2:4 sparse FF2 contract (SMFMAC) ----------------------------------------------

def test_ffn_contract_fp8_sparse(pk, orc):
    """The expand epilogue 7 output (2:4 compressed e4m3) feeds the sparse contract."""
    note("ffn_contract_fp8_sparse")
    rows = 272
    rng = np.random.default_rng(161)
    dense = orc.quantize_fp8_static((rng.standard_normal((rows, 4096)) * 2).astype(np.float16), 16.0)
    data, meta = orc.compress_24(dense)
    w = weights(1024, 4096, 162)
    wq, ws = orc.pack_fp8_rows(w)
    residual = acts(rows, 1024, 163, outliers=False)
    buf = np.concatenate([data.ravel(), meta.ravel()])
    out = dev(residual.copy())
    pk.call("pk_ffn_contract_fp8_sparse", dev(buf), dev(wq), dev(ws), out, rows, 4096)
    ref = orc.epilogue(orc.gemm_e4m3(orc.decompress_24(data, meta), wq), 8, ws, in_scale=1.0 / 16.0,
                       residual=residual)
    assert_close(host(out).astype(np.float32), ref.astype(np.float32))  # 1e-2 * RMS(output)
    delta_ref = ref.astype(np.float32) - residual.astype(np.float32)
    delta_got = host(out).astype(np.float32) - residual.astype(np.float32)
    assert_close(delta_got, delta_ref, tol=2e-2)  # the update alone


@pytest.mark.parametrize("int8", [False, True])
def test_joint_scan(pk, orc, int8):
    """Whole utterance through repeated scans (the prediction vector redrawn
    after each token, as the prediction network would) against the oracle loop
    over the oracle's per-frame scores."""
    note(f"joint scan int8={int8}")
    T, D, hidden, frames = 1025, 5, 640, 160
    outputs = T + D
    rng = np.random.default_rng(150 + int8)
    w = (rng.standard_normal((outputs, hidden)) * 0.05).astype(np.float16)
    bias = (rng.standard_normal(outputs) * 0.1).astype(np.float32)
    bias[T - 1] += 2.2  # blank-dominated frames, as in real audio
    enc = (rng.standard_normal((frames, hidden)) * 0.5).astype(np.float16)
    if int8:
        wq, ws = orc.quantize_int8_rows(w)
        d_w, d_ws = dev(wq), dev(ws)
        score = lambda t, pred: orc.joint_scores_i8(wq, ws, bias, enc[t], pred)
    else:
        d_w, d_ws = dev(w), None
        score = lambda t, pred: orc.joint_scores_f16(w, bias, enc[t], pred)
    d_bias, d_enc = dev(bias), dev(enc)
    state = torch.zeros(4, dtype=torch.int32, device="cuda")
    work = torch.zeros(2304, dtype=torch.int32, device="cuda")
    frame = symbols = 0
    tokens, scans = [], 0
    while True:
        pred = (rng.standard_normal(hidden) * 0.3).astype(np.float32)
        ref = orc.joint_scan(lambda t: score(t, pred), frames, frame, symbols)
        state[0], state[1] = frame, symbols
        pk.call("pk_joint_scan", d_w, int(int8), d_ws, d_bias, d_enc, dev(pred), outputs, hidden, T, D,
                frames, hidden, 10, state, work)
        got = tuple(int(v) for v in host(state))
        assert got == ref, f"scan {scans}: {got} != {ref}"
        scans += 1
        frame, symbols, tok, _ = got
        if tok < 0:
            break
        tokens.append(tok)
    note(f"joint scan: {scans} scans, {len(tokens)} tokens")
    assert 3 <= len(tokens) < frames


# ---- .pkl4 load-time derivation ----------------------------------------------------------

@pytest.mark.parametrize("fmt", ["fp16", "fp8", "int8", "int4", "g128"])
def test_artifact_derive_linear(pk, orc, fmt, tmp_path):
    """A linear read from a .pkl4 artifact, uploaded and packed on the GPU,
    equals the oracle's packer applied to the artifact's padded fp16 matrix."""
    sys.path.insert(0, __import__("os").path.dirname(__file__))
    import pkl4_writer

    note(f"artifact derive {fmt}")
    rng = np.random.default_rng(160)
    wsrc = rng.standard_normal((300, 200)) * 0.02
    path = pkl4_writer.write(tmp_path / "d.pkl4", [("encoder.layers.3.feed_forward2.linear1.weight", "linear", wsrc)])
    art = pk.Artifact(str(path))
    idx = art.find("encoder.layers.3.feed_forward2.linear1.weight")
    n, k = art.tensor(idx)["physical_shape"]
    padded = np.zeros((n, k), np.float16)
    padded[:300, :200] = wsrc.astype(np.float16)
    staging = np.empty(n * k * 2, np.uint8)
    d16 = empty((n, k), torch.float16)
    if fmt == "fp16":
        art.derive_linear(idx, pk.DERIVE_FP16, staging, d16)
        assert np.array_equal(host(d16).view(np.uint16), padded.view(np.uint16))
    elif fmt in ("fp8", "int8"):
        q = empty((n, k), torch.uint8 if fmt == "fp8" else torch.int8)
        sc = empty((n,), torch.float32)
        art.derive_linear(idx, pk.DERIVE_FP8_ROWS if fmt == "fp8" else pk.DERIVE_INT8_ROWS, staging, d16, q, sc)
        rq, rs = orc.pack_fp8_rows(padded) if fmt == "fp8" else orc.pack_int8_rows(padded)
        assert np.array_equal(host(q).view(np.uint8), np.asarray(rq).view(np.uint8))
        assert np.array_equal(host(sc), rs)
    elif fmt == "int4":
        q = empty((n, k // 2), torch.uint8)
        sc = empty((n,), torch.float32)
        art.derive_linear(idx, pk.DERIVE_INT4_ROWS, staging, d16, q, sc)
        rq, rs = orc.pack_int4_rows(padded)
        assert np.array_equal(host(q), rq) and np.array_equal(host(sc), rs)
    else:
        q = empty((n, k // 8), torch.int32)
        sc = empty((n, k // 128), torch.float16)
        z = empty((n, k // 128), torch.float16)
        art.derive_linear(idx, pk.DERIVE_INT4_G128, staging, d16, q, sc, z)
        rq, rs, rz = orc.pack_int4_g128(padded)
        assert np.array_equal(host(q).view(np.uint32), rq)
        assert np.array_equal(host(sc).view(np.uint16), rs.view(np.uint16))
        assert np.array_equal(host(z).view(np.uint16), rz.view(np.uint16))
    art.close()


# ---- TDT greedy decode ---------------------------------------------------------------------

def decode_case(H, T, D, frames, seed, int8):
    rng = np.random.default_rng(seed)
    f16 = lambda *s, sc=0.05: (rng.standard_normal(s) * sc).astype(np.float16)
    f32 = lambda *s, sc=0.1: (rng.standard_normal(s) * sc).astype(np.float32)
    lstm = (f16(4 * H, H), f16(4 * H, H), f32(4 * H), f32(4 * H), f16(4 * H, H), f16(4 * H, H), f32(4 * H), f32(4 * H))
    proj = (f16(H, H, sc=0.1), f32(H))
    wj = f16(T + D, H, sc=0.08)
    bj = f32(T + D)
    bj[T - 1] += 2.0 * np.sqrt(H / 640)  # blank-dominated frames, as in real audio
    enc = f16(frames, H, sc=0.5)
    emb = f16(T - 1, H, sc=0.5)
    return lstm, proj, wj, bj, enc, emb


@pytest.mark.parametrize("H,int8", [(640, False), (640, True), (128, False)])
def test_tdt_decode(pk, orc, H, int8):
    """The whole utterance decoded in one persistent launch: tokens, final
    frame and final prediction vector against the oracle's decode loop."""
    T, D, frames = 1025, 5, 96
    note(f"tdt decode H={H} int8={int8}")
    lstm, proj, wj, bj, enc, emb = decode_case(H, T, D, frames, 180 + H + int8, int8)
    if int8:
        wq, ws = orc.quantize_int8_rows(wj)
        joint = (wq, ws, bj)
    else:
        joint = (wj, None, bj)
    ref_toks, ref_frame, ref_pred = orc.tdt_decode(enc, emb, lstm, proj, joint, T, D)
    assert 3 <= len(ref_toks) <= 10 * frames, len(ref_toks)
    d = [dev(a) for a in lstm]
    cap = frames * 10
    toks = torch.zeros(cap, dtype=torch.int32, device="cuda")
    res = torch.zeros(4, dtype=torch.int32, device="cuda")
    wbytes = pk.lib.pk_tdt_decode_workspace_bytes(H)
    work = torch.zeros(wbytes // 4, dtype=torch.int32, device="cuda")
    pk.call("pk_tdt_decode", dev(enc), frames, H, dev(emb), d[0], d[1], d[2], d[3], d[4], d[5], d[6], d[7],
            dev(proj[0]), dev(proj[1]), dev(joint[0]), int(int8), None if joint[1] is None else dev(joint[1]),
            dev(bj), H, T, D, 10, toks, cap, res, work, wbytes)
    count, frame, status, steps = (int(v) for v in host(res))
    note(f"tdt decode: {count} tokens, {steps} joint steps, status {status}")
    assert status == 0
    assert count == len(ref_toks) and frame == ref_frame
    assert np.array_equal(host(toks)[:count], ref_toks)
    pred = host(work).view(np.float32)[1032 + 8 * H:1032 + 9 * H]  # state after the 1032-word barrier area
    assert np.max(np.abs(pred - ref_pred)) <= 1e-4 * max(1.0, float(np.max(np.abs(ref_pred))))


def run_long_decode(pk, orc, H, int8, frames, seed, T=1025, D=5):
    """The long-request decode on the GPU against the oracle's long decode on
    the same input table.  At frames >= 1024 it runs through the decoder.rs
    launch mirror (which must pick the long form), below that the table and
    pk_tdt_decode_long are called directly."""
    lstm, proj, wj, bj, enc, emb = decode_case(H, T, D, frames, seed, int8)
    if int8:
        wq, ws = orc.quantize_int8_rows(wj)
        joint = (wq, ws, bj)
    else:
        joint = (wj, None, bj)
    d = [dev(a) for a in lstm]
    cap = frames * 10
    toks = torch.zeros(cap, dtype=torch.int32, device="cuda")
    res = torch.zeros(4, dtype=torch.int32, device="cuda")
    work = torch.zeros(pk.lib.pk_tdt_decode_workspace_bytes(H) // 4, dtype=torch.int32, device="cuda")
    wbytes = work.numel() * 4
    table_d = torch.zeros((T - 1, 4 * H), dtype=torch.float16, device="cuda")
    js = None if joint[1] is None else dev(joint[1])
    if frames >= pk.LONG_DECODE_MIN_FRAMES:
        form = pk.launch_decode(dev(enc), frames, (dev(emb),) + tuple(d), (dev(proj[0]), dev(proj[1])),
                                (dev(joint[0]), dev(bj)), toks, res, work, input_table=table_d, joint_int8=int8,
                                joint_scales=js, hidden=H, token_outputs=T, durations=D)
        assert form == "long"
    else:
        pk.launch_linear(dev(emb), d[0], None, None, table_d, T - 1, 4 * H, H)
        pk.call("pk_tdt_decode_long", dev(enc), frames, H, table_d, d[1], d[2], d[3], d[4], d[5], d[6], d[7],
                dev(proj[0]), dev(proj[1]), dev(joint[0]), int(int8), js, dev(bj), H, T, D, 10, toks, cap, res, work,
                wbytes)
    table = host(table_d)
    # the table is the fp16 linear of the embedding with W_ih0: fp32 accumulation (error <= H * 2^-24 * sum|e w|)
    # and one fp16 rounding (half an ulp: 2^-11 relative, 2^-25 absolute below the normal range)
    e64, w64 = emb.astype(np.float64), lstm[0].astype(np.float64)
    exact = e64 @ w64.T
    bound = 2.0 ** -11 * np.abs(exact) + 2.0 ** -25 + H * 2.0 ** -24 * (np.abs(e64) @ np.abs(w64).T)
    err = np.abs(table.astype(np.float64) - exact)
    assert np.all(err <= bound * (1 + 1e-9)), float((err / bound).max())
    ref = orc.tdt_decode_long(enc, table, lstm[1:], proj, joint, T, D)
    return (toks, res, work), ref


@pytest.mark.parametrize("form", ["long", "fp16"])
def test_tdt_decode_full_length(pk, orc, form):
    """An hour of synthetic audio (45000 frames, H = 640, INT8 joint) in one
    launch, twice: tens of thousands of barrier epochs (tag reuse, slot
    parity, the joint rounds' windows) must end with status 0 and identical
    tokens.  The greedy decode is causal (a decision at frame f reads encoder
    rows <= f and the tokens before it), so the full decode's tokens begin
    with exactly the oracle's decode of the first 1100 frames."""
    H, T, D, frames, head = 640, 1025, 5, 45000, 1100
    note(f"tdt decode full length form={form} frames={frames}")
    lstm, proj, wj, bj, enc, emb = decode_case(H, T, D, frames, 977, True)
    bj[T - 1] += 0.8  # about a token every 5 frames, as in speech; duration 0 rare, 1 preferred
    bj[T] -= 3.0
    bj[T + 1] += 0.5
    wq, ws = orc.quantize_int8_rows(wj)
    d = [dev(a) for a in lstm]
    cap = frames * 10
    work = torch.zeros(pk.lib.pk_tdt_decode_workspace_bytes(H) // 4, dtype=torch.int32, device="cuda")
    table_d = torch.zeros((T - 1, 4 * H), dtype=torch.float16, device="cuda")
    enc_d, emb_d, wq_d, ws_d, bj_d = dev(enc), dev(emb), dev(wq), dev(ws), dev(bj)
    runs = []
    for _ in range(2):
        toks = torch.zeros(cap, dtype=torch.int32, device="cuda")
        res = torch.zeros(4, dtype=torch.int32, device="cuda")
        if form == "long":
            got = pk.launch_decode(enc_d, frames, (emb_d,) + tuple(d), (dev(proj[0]), dev(proj[1])), (wq_d, bj_d), toks, res,
                                   work, input_table=table_d, joint_int8=True, joint_scales=ws_d, hidden=H,
                                   token_outputs=T, durations=D)
            assert got == "long"
        else:
            pk.call("pk_tdt_decode", enc_d, frames, H, emb_d, *d, dev(proj[0]), dev(proj[1]), wq_d, 1, ws_d, bj_d, H, T,
                    D, 10, toks, cap, res, work, work.numel() * 4)
        count, frame, status, steps = (int(v) for v in host(res))
        note(f"  {count} tokens, {steps} joint steps, final frame {frame}, status {status}")
        assert status == 0 and frame >= frames and frames // 50 <= count <= cap and steps >= count
        runs.append(host(toks)[:count])
    assert np.array_equal(runs[0], runs[1])
    assert np.all((runs[0] >= 0) & (runs[0] < T - 1))
    joint = (wq, ws, bj)
    if form == "long":
        ref, _, _ = orc.tdt_decode_long(enc[:head], host(table_d), lstm[1:], proj, joint, T, D)
    else:
        ref, _, _ = orc.tdt_decode(enc[:head], emb, lstm, proj, joint, T, D)
    assert len(ref) >= 20
    assert np.array_equal(runs[0][:len(ref)], ref)


@pytest.mark.parametrize("H,int8,frames", [(640, False, 1100), (640, True, 96), (128, True, 96), (128, False, 96)])
def test_tdt_decode_long(pk, orc, H, int8, frames):
    """decoder.cu:452-784 long-request decode (INT8 recurrent weights derived
    in the launch, INT8 hidden states, layer-0 input table): tokens and final
    frame exact, final prediction within 1e-4 of the oracle's."""
    note(f"tdt decode long H={H} int8={int8} frames={frames}")
    (toks, res, work), (ref_toks, ref_frame, ref_pred) = run_long_decode(pk, orc, H, int8, frames, 380 + H + int8)
    assert 3 <= len(ref_toks) <= 10 * frames, len(ref_toks)
    count, frame, status, steps = (int(v) for v in host(res))
    note(f"tdt decode long: {count} tokens, {steps} joint steps, status {status}")
    got = host(toks)[:min(count, len(toks))]
    n = min(len(got), len(ref_toks))
    diff = np.nonzero(got[:n] != ref_toks[:n])[0]
    note(f"  oracle {len(ref_toks)} tokens; first divergence at token {int(diff[0]) if len(diff) else n}")
    assert status == 0
    assert count == len(ref_toks) and frame == ref_frame
    assert np.array_equal(host(toks)[:count], ref_toks)
    pred = host(work).view(np.float32)[1032 + 8 * H:1032 + 9 * H]
    assert np.max(np.abs(pred - ref_pred)) <= 1e-4 * max(1.0, float(np.max(np.abs(ref_pred))))
