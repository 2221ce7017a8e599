"""The FF hidden written by the expand in the form its contract reads, at
T = 45000 (the benchmark's stack; no re-quantization pass between them):

* static INT8 at the x16 hidden scale (epilogue 7, rne(clamp(fp16(SiLU(v)) *
  16, +-127)), linear.cu:549-560 applied to the encoder.cu:1010-1025 hidden)
  from FP8, INT8 and INT4-g128 x INT8 expands, read by INT8 and INT4-g128
  contracts at input scale 1/16;
* e4m3 x16 (the reference's own hidden) read by the INT4-g128 contract as
  pk_gemm format 8: the packed weights expanded per call to e4m3 (q - z)
  (pk_expand_int4_g128_e4m3, exact), one f8f6f4 MFMA per 128-K group.

Tolerances: the INT8 hidden's codes equal the oracle's except where the
device exp moves an fp16 rounding boundary (>= 99 % equal, all within one
code); format 8's fp32 outputs within 1e-2 * RMS of the oracle (it sums a
group in fp32 in the MFMA's order, the oracle in double) -- and in fact
within 1e-4 -- and its fp16 + residual outputs in the stated form.
"""
import numpy as np
import pytest

from test_gpu_fullsize import assert_close, host, note, rows_of, sample_rows

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

D, FF = 1024, 4096
T = 45000


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


def g128(pk, n, k, gen):
    w16 = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).half()
    q = torch.empty((n, k // 8), dtype=torch.int32, device="cuda")
    s = torch.empty((n, k // 128), dtype=torch.float16, device="cuda")
    z = torch.empty((n, k // 128), dtype=torch.float16, device="cuda")
    pk.call("pk_pack_int4_g128", w16, n, k, q, s, z)
    return q, s, z


@pytest.mark.parametrize("n,k", [(D, FF), (FF, D), (256, 128)])
def test_expand_int4_g128_e4m3(pk, orc, n, k):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(n * 3 + k)
    q, s, z = g128(pk, n, k, gen)
    out = torch.empty((n, k), dtype=torch.uint8, device="cuda")
    st = torch.empty((k // 128, n), dtype=torch.float16, device="cuda")
    note(f"expand_int4_g128_e4m3 n={n} k={k}")
    pk.call("pk_expand_int4_g128_e4m3", q, z, s, n, k, out, st)
    assert np.array_equal(host(st).view(np.uint16), host(s).view(np.uint16).T)
    b = host(q).view(np.uint8).reshape(n, -1, 4).astype(np.int64)
    lv = np.concatenate([b & 15, b >> 4], axis=2).reshape(n, -1)
    want = lv - np.repeat(host(z).astype(np.int64), 128, axis=1)
    assert np.array_equal(orc.e4m3_table()[host(out)], want.astype(np.float32))


@pytest.mark.parametrize("fmt", ["fp8", "int8", "int4g128"])
def test_expand_static_int8_hidden(pk, orc, fmt):
    """FF1 expand 1024 -> 4096 at T = 45000 writing the INT8 hidden."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(900 + len(fmt))
    x = torch.randn((T, D), generator=gen, device="cuda").half()
    w16 = (torch.randn((FF, D), generator=gen, device="cuda") * 0.05).half()
    xq = torch.empty((T, D), dtype=torch.uint8 if fmt == "fp8" else torch.int8, device="cuda")
    xs = torch.empty(T, dtype=torch.float32, device="cuda")
    pk.call("pk_quantize_rows", 0 if fmt == "fp8" else 1, x, xq, xs, T, T, D)
    out = torch.empty((T, FF), dtype=torch.int8, device="cuda")
    idx = sample_rows(T, 61 + len(fmt))
    if fmt == "int4g128":
        q, s, z = g128(pk, FF, D, gen)
        f = pk.FMT_G128A8
        pk.gemm(f, 7, xq, q, T, FF, D, out, row_scales=xs, g_scales=s, g_zeros=z)
        acc = orc.gemm_g128_a8(rows_of(xq, idx), rows_of(xs, idx), host(q).view(np.uint32), host(s), host(z))
        ref = orc.epilogue(acc, 9, np.ones(FF, np.float32))
    else:
        wq = torch.empty((FF, D), dtype=xq.dtype, device="cuda")
        ws = torch.empty(FF, dtype=torch.float32, device="cuda")
        pk.call("pk_pack_fp8_rows" if fmt == "fp8" else "pk_pack_int8_rows", w16, FF, D, wq, ws)
        f = pk.FMT_FP8 if fmt == "fp8" else pk.FMT_I8
        pk.gemm(f, 7, xq, wq, T, FF, D, out, w_scales=ws, row_scales=xs)
        acc = orc.gemm_e4m3(rows_of(xq, idx), host(wq)) if fmt == "fp8" else \
            orc.gemm_i8(rows_of(xq, idx), host(wq)).astype(np.float32)
        ref = orc.epilogue(acc, 9, host(ws), row_scales=rows_of(xs, idx))
    note(f"static INT8 hidden from {fmt} expand T={T} tile={pk.gemm_tile(f, 7, T, FF)}")
    got = rows_of(out, idx).astype(np.int32)
    want = ref.view(np.int8).astype(np.int32)
    assert np.mean(got == want) >= 0.99, np.mean(got == want)
    assert np.all(np.abs(got - want) <= 1)
    assert (np.abs(want) > 16).mean() > 0.01  # the codes span more than the unit range


def test_int8_contract_on_static_hidden(pk, orc):
    """INT8 and INT4-g128 x INT8 contracts (fp16 + 0.5 residual) reading the
    static INT8 hidden at input scale 1/16, no row scales: exact accumulators,
    fp16 outputs bit for bit."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(931)
    h = torch.randint(-127, 128, (T, FF), generator=gen, device="cuda", dtype=torch.int8)
    idx = sample_rows(T, 71)
    w16 = (torch.randn((D, FF), generator=gen, device="cuda") * 0.02).half()
    wq = torch.empty((D, FF), dtype=torch.int8, device="cuda")
    ws = torch.empty(D, dtype=torch.float32, device="cuda")
    pk.call("pk_pack_int8_rows", w16, D, FF, wq, ws)
    state = torch.randn((T, D), generator=gen, device="cuda").half()
    before = rows_of(state, idx)
    pk.gemm(pk.FMT_I8, pk.EPI_F16, h, wq, T, D, FF, state, w_scales=ws, in_scale=1.0 / 16, residual=state,
            out_scale=0.5, res_scale=1.0)
    ref = orc.epilogue(orc.gemm_i8(rows_of(h, idx), host(wq)).astype(np.float32), 2, host(ws), in_scale=1.0 / 16,
                       residual=before)
    assert np.array_equal(rows_of(state, idx).view(np.uint16), ref.view(np.uint16))
    q, s, z = g128(pk, D, FF, gen)
    before = rows_of(state, idx)
    pk.gemm(pk.FMT_G128A8, pk.EPI_F16, h, q, T, D, FF, state, in_scale=1.0 / 16, residual=state, out_scale=0.5,
            res_scale=1.0, g_scales=s, g_zeros=z)
    xs = np.full(len(idx), 1.0 / 16, np.float32)
    acc = orc.gemm_g128_a8(rows_of(h, idx), xs, host(q).view(np.uint32), host(s), host(z))
    ref = orc.epilogue(acc, 2, np.ones(D, np.float32), residual=before)
    assert np.array_equal(rows_of(state, idx).view(np.uint16), ref.view(np.uint16))


def test_g128_f8_contract(pk, orc):
    """Format 8 on the e4m3 x16 hidden: fp32 outputs, then the stack's
    fp16 + 0.5 residual epilogue, T = 45000, N = 1024, K = 4096, plus the FF1
    shape with the fp16 epilogue."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(941)
    idx = sample_rows(T, 81)
    for n, k in ((D, FF), (FF, D)):
        h = (torch.randn((T, k), generator=gen, device="cuda") * 2).to(torch.float8_e4m3fn).view(torch.uint8)
        q, s, z = g128(pk, n, k, gen)
        we = torch.empty((n, k), dtype=torch.uint8, device="cuda")
        st = torch.empty((k // 128, n), dtype=torch.float16, device="cuda")
        pk.call("pk_expand_int4_g128_e4m3", q, z, s, n, k, we, st)
        note(f"g128 f8 n={n} k={k} T={T} tile={pk.gemm_tile(pk.FMT_G128F8, pk.EPI_F32, T, n)}")
        out = torch.empty((T, n), dtype=torch.float32, device="cuda")
        pk.gemm(pk.FMT_G128F8, pk.EPI_F32, h, we, T, n, k, out, in_scale=1.0 / 16, g_scales=st)
        ref = orc.gemm_g128_f8(rows_of(h, idx), host(q).view(np.uint32), host(s), host(z)) * np.float32(1.0 / 16)
        got = rows_of(out, idx)
        assert_close(got, ref, what=f"g128 f8 fp32 n={n}")
        assert_close(got, ref, tol=1e-4, what=f"g128 f8 fp32 n={n} (tight)")
        if n == D:
            state = torch.randn((T, D), generator=gen, device="cuda").half()
            before = rows_of(state, idx)
            pk.gemm(pk.FMT_G128F8, pk.EPI_F16, h, we, T, n, k, state, in_scale=1.0 / 16, residual=state,
                    out_scale=0.5, res_scale=1.0, g_scales=st)
            ref16 = orc.epilogue(ref * np.float32(16.0), 2, np.ones(n, np.float32), in_scale=1.0 / 16,
                                 residual=before)
            after = rows_of(state, idx)
            assert_close(after, ref16, what="g128 f8 + residual (output)")
            d_ref = ref16.astype(np.float32) - before.astype(np.float32)
            assert_close(after.astype(np.float32) - before.astype(np.float32), d_ref, tol=2e-2,
                         what="g128 f8 + residual (update)")
        else:
            o16 = torch.empty((T, n), dtype=torch.float16, device="cuda")
            pk.gemm(pk.FMT_G128F8, pk.EPI_F16, h, we, T, n, k, o16, in_scale=1.0 / 16, g_scales=st)
            assert_close(rows_of(o16, idx), ref, what="g128 f8 fp16")
        del h, we, out
    torch.cuda.empty_cache()
