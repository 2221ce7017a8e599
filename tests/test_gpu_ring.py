"""Parity of the one-tile-per-workgroup ring GEMM (grids of at most one tile
per CU: BASELINE config 1, the T = 750 INT4-g128 linears) against the CPU
oracle, through the C ABI: INT8 accumulators and INT4-g128 x INT8 outputs
bit for bit, FP8 / INT4-g128 x fp16 outputs within 1e-2 x RMS.  Shapes cover
a single K-step, fewer K-steps than ring stages, many more, and ragged M."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


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


def note(msg):
    print(f"[gpu-ring] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(t):
    torch.cuda.synchronize()
    a = t.cpu()
    if a.dtype == torch.float16:
        return a.view(torch.int16).numpy().view(np.float16)
    return a.numpy()


def assert_close(got, ref, tol=1e-2):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    assert np.isfinite(got).all()
    assert np.max(np.abs(got - ref)) <= tol * rms


def ring(pk, fmt, epi, m, n):
    rows, cols, stages = pk.gemm_tile(fmt, epi, m, n, stages=True)
    assert stages > 2, (m, n, rows, stages)
    return rows


@pytest.mark.parametrize("m,n,k", [(750, 4096, 1024), (97, 1024, 4096), (1, 640, 1024), (33, 256, 128), (200, 1024, 512),
                                   (750, 1536, 1024), (700, 1536, 384)])
def test_ring_int8_accumulators_exact(pk, orc, m, n, k):
    rows = ring(pk, pk.FMT_I8, pk.EPI_I32, m, n)
    note(f"int8 m={m} n={n} k={k} ring rows={rows}")
    rng = np.random.default_rng(m + n + k)
    x = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    pk.call("pk_linear_int8_accumulate", dev(x), dev(w), acc, m, n, k)
    assert np.array_equal(host(acc), orc.gemm_i8(x, w))


def test_ring_int8_dyn_config1(pk, orc):
    """BASELINE config 1's GEMM (750 x 1024 -> 4096, per-token INT8, fp32 out)."""
    m, n, k = 750, 4096, 1024
    ring(pk, pk.FMT_I8, pk.EPI_F32, m, n)
    rng = np.random.default_rng(0x5EED0001)
    x = (rng.standard_normal((m, k))).astype(np.float16)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    xq, xs = orc.quantize_int8_rows(x)
    wq, ws = orc.pack_int8_rows(w)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    pk.call("pk_linear_int8_dyn", dev(xq), dev(xs), dev(wq), dev(ws), None, out, 1, m, n, k)
    ref = (orc.gemm_i8(xq, wq).astype(np.float32) * xs[:, None]).astype(np.float32) * ws[None, :]
    assert np.array_equal(host(out), ref.astype(np.float32))


@pytest.mark.parametrize("m,n,k,ldo", [(97, 1040, 512, 1040), (750, 4096, 128, 4112), (5, 272, 1024, 304)])
def test_ring_fp32_staged_ragged(pk, orc, m, n, k, ldo):
    """fp32 ring outputs go through per-wave LDS and whole-line stores: ragged
    M, N not a multiple of the 128-column tile, a row stride beyond N (the
    columns past N stay untouched), one K-step; INT8 bit for bit."""
    rows = ring(pk, pk.FMT_I8, pk.EPI_F32, m, n)
    note(f"int8 fp32 staged m={m} n={n} k={k} ldo={ldo} ring rows={rows}")
    rng = np.random.default_rng(m * 3 + n + k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    xq, xs = orc.quantize_int8_rows(x)
    wq, ws = orc.pack_int8_rows(w)
    out = torch.full((m, ldo), -7.0, dtype=torch.float32, device="cuda")
    pk.gemm(pk.FMT_I8, pk.EPI_F32, dev(xq), dev(wq), m, n, k, out, w_scales=dev(ws), row_scales=dev(xs), ldo=ldo)
    got = host(out)
    ref = (orc.gemm_i8(xq, wq).astype(np.float32) * xs[:, None]).astype(np.float32) * ws[None, :]
    assert np.array_equal(got[:, :n], ref.astype(np.float32))
    assert np.all(got[:, n:] == -7.0)


@pytest.mark.parametrize("m,n,k", [(750, 4096, 1024), (300, 1024, 4096), (45, 3072, 1024), (750, 1536, 1024)])
def test_ring_fp8_epilogues(pk, orc, m, n, k):
    rows = ring(pk, pk.FMT_FP8, pk.EPI_F16, m, n)
    note(f"fp8 m={m} n={n} k={k} ring rows={rows}")
    rng = np.random.default_rng(7 * m + n)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    xq, xs = orc.quantize_fp8_rows(x)
    wq, ws = orc.pack_fp8_rows(w)
    acc = orc.gemm_e4m3(xq, wq)
    o32 = torch.empty((m, n), dtype=torch.float32, device="cuda")
    pk.gemm(pk.FMT_FP8, pk.EPI_F32, dev(xq), dev(wq), m, n, k, o32, w_scales=dev(ws), row_scales=dev(xs))
    assert_close(host(o32), acc * xs[:, None] * ws[None, :])
    o8 = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    pk.gemm(pk.FMT_FP8, pk.EPI_F8, dev(xq), dev(wq), m, n, k, o8, w_scales=dev(ws), row_scales=dev(xs))
    ref8 = orc.epilogue(acc, 1, ws, row_scales=xs)
    got8 = host(o8)
    t = orc.e4m3_table().astype(np.float64)
    assert np.mean(got8 == ref8) >= 0.99
    assert np.all(np.abs(t[got8] - t[ref8]) <= np.abs(t[ref8]) / 8 + 2.0 ** -9 + 1e-12)
    res = (rng.standard_normal((m, n))).astype(np.float16)
    st = dev(res.copy())
    pk.gemm(pk.FMT_FP8, pk.EPI_F16, dev(xq), dev(wq), m, n, k, st, w_scales=dev(ws), row_scales=dev(xs), residual=st,
            out_scale=0.5, res_scale=1.0)
    ref = orc.epilogue(acc, 2, ws, row_scales=xs, residual=res)
    assert_close(host(st).astype(np.float32) - res.astype(np.float32), ref.astype(np.float32) - res.astype(np.float32),
                 tol=2e-2)


# shapes whose 32-row ring tiles split K in four parts within the workgroup
SPLIT_SHAPES = {(750, 1024, 4096), (97, 1024, 4096), (45, 1024, 1280), (33, 256, 1024)}


@pytest.mark.parametrize("m,n,k", [(750, 1024, 4096), (97, 1024, 4096), (750, 4096, 1024), (5, 256, 256),
                                   (45, 1024, 1280), (33, 256, 1024)])
def test_ring_int4g128_a8_exact(pk, orc, m, n, k):
    """INT4-g128 x INT8: fp32 (and fp16 + residual) outputs bit for bit; the
    ring loads each tile's group tables once and indexes them by K-step.  The
    split-K shapes (10 groups in 4 parts: runs of 2, 3, 2, 3; 8 in 4)
    compare with the oracle's matching association of the group sum."""
    rows = ring(pk, pk.FMT_G128A8, pk.EPI_F32, m, n)
    note(f"g128 a8 m={m} n={n} k={k} ring rows={rows}")
    rng = np.random.default_rng(11 * m + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    q, s, z = orc.pack_int4_g128(w)
    x = rng.standard_normal((m, k)).astype(np.float16)
    xq, xs = orc.quantize_int8_rows(x)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    pk.call("pk_linear_int4g128_a8", dev(xq), dev(xs), dev(q), dev(s), dev(z), None, out, 1, m, n, k)
    parts = pk.gemm_k_split(pk.FMT_G128A8, pk.EPI_F32, m, n, k)
    assert parts == (4 if (m, n, k) in SPLIT_SHAPES else 1), parts
    ref = orc.gemm_g128_a8(xq, xs, q, s, z, parts=parts)
    assert np.array_equal(host(out), ref)
    res = rng.standard_normal((m, n)).astype(np.float16)
    st = dev(res.copy())
    pk.gemm(pk.FMT_G128A8, pk.EPI_F16, dev(xq), dev(q), m, n, k, st, row_scales=dev(xs), residual=st, out_scale=0.5,
            res_scale=1.0, g_scales=dev(s), g_zeros=dev(z))
    want = orc.epilogue(ref, 2, np.ones(n, np.float32), residual=res)
    assert np.array_equal(host(st).view(np.uint16), want.view(np.uint16))
    if (m, n, k) in SPLIT_SHAPES:
        # the SiLU -> e4m3 epilogue on the split path (one e4m3 step on < 1 % of codes)
        o8 = torch.empty((m, n), dtype=torch.uint8, device="cuda")
        pk.gemm(pk.FMT_G128A8, pk.EPI_F8, dev(xq), dev(q), m, n, k, o8, row_scales=dev(xs), g_scales=dev(s),
                g_zeros=dev(z))
        ref8 = orc.epilogue(ref, 1, np.ones(n, np.float32))
        got8 = host(o8)
        t = orc.e4m3_table().astype(np.float64)
        assert np.mean(got8 == ref8) >= 0.99
        assert np.all(np.abs(t[got8] - t[ref8]) <= np.abs(t[ref8]) / 8 + 2.0 ** -9 + 1e-12)


@pytest.mark.parametrize("m,n,k", [(750, 1024, 4096), (750, 4096, 1024), (97, 1024, 4096), (45, 1024, 1280)])
def test_ring_int4g128_a16(pk, orc, m, n, k):
    ring(pk, pk.FMT_G128A16, pk.EPI_F32, m, n)
    note(f"g128 a16 m={m} n={n} k={k} split={pk.gemm_k_split(pk.FMT_G128A16, pk.EPI_F32, m, n, k)}")
    rng = np.random.default_rng(13 * m + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    q, s, z = orc.pack_int4_g128(w)
    x = rng.standard_normal((m, k)).astype(np.float16)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    pk.call("pk_linear_int4g128", dev(x), dev(q), dev(s), dev(z), None, out, 1, m, n, k)
    assert_close(host(out), orc.gemm_g128_a16(x, q, s, z))
