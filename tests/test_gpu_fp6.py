"""INT4 codes as FP6 e3m2 on the f8f6f4 MFMA (pk_gemm format 9), against the
INT8 path on the same codes, bit for bit:

* pk_layer_norm_quantize_int4_fp6 writes the oracle's FP6 chunk form
  (pk_oracle.fp6_chunks) of the codes pk_layer_norm_quantize_int4_codes
  writes, with the same scales, on sampled and padding rows;
* pk_unpack_int4_fp6 writes the FP6 chunk form of pk_unpack_int4's codes;
* format 9 with fp32 outputs gives exactly the int32 accumulators of format 1
  on the int8 codes (FP6 products of codes are exact, and fp32 sums of
  integers below 2^24 are exact), ragged and full-size shapes;
* pk_ffn_expand_int4_sparse_fp6 writes exactly the bytes (2:4 data and
  metadata) of pk_ffn_expand_int4_sparse_codes, up to T = 45000.
"""
import numpy as np
import pytest

from test_gpu_fullsize import host, note, rows_of, sample_rows
from test_gpu_refplan import ln_params, padded

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

D, FF = 1024, 4096


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


def int4_weights(pk, gen, n=FF, k=D):
    w16 = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).half()
    wq = torch.empty((n, k // 2), dtype=torch.uint8, device="cuda")
    ws = torch.empty(n, dtype=torch.float32, device="cuda")
    pk.call("pk_pack_int4_rows", w16, n, k, wq, ws)
    wc = torch.empty((n, k), dtype=torch.int8, device="cuda")
    pk.call("pk_unpack_int4", wq, wc, n * k)
    wf = torch.full((n, k), 0x5A, dtype=torch.uint8, device="cuda")
    pk.call("pk_unpack_int4_fp6", wq, wf, n * k)
    return wq, ws, wc, wf


def codes_and_fp6(pk, gen, t, pad):
    x = (torch.randn((pad, D), generator=gen, device="cuda") * 2).half()
    g, b = ln_params(gen)
    xc = torch.full((pad, D), 5, dtype=torch.int8, device="cuda")
    xcs = torch.empty(pad, dtype=torch.float32, device="cuda")
    xf = torch.full((pad, D), 0x5A, dtype=torch.uint8, device="cuda")
    xfs = torch.empty(pad, dtype=torch.float32, device="cuda")
    pk.call("pk_layer_norm_quantize_int4_codes", x, g, b, xc, xcs, t, pad, 1e-5)
    pk.call("pk_layer_norm_quantize_int4_fp6", x, g, b, xf, xfs, t, pad, 1e-5)
    return xc, xcs, xf, xfs


@pytest.mark.parametrize("t", [300, 7500, 45000])
def test_fp6_producer_and_weights(pk, orc, t):
    pad = padded(t) + 16
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2600 + t)
    note(f"int4 fp6 producer T={t} padded={pad}")
    xc, xcs, xf, xfs = codes_and_fp6(pk, gen, t, pad)
    assert torch.equal(xcs, xfs)
    idx = np.union1d(sample_rows(pad, t + 9, per_strip=2), np.arange(t - 2, pad))
    assert np.array_equal(rows_of(xf, idx), orc.fp6_chunks(rows_of(xc, idx)))
    assert np.all(rows_of(xf, np.arange(t, pad)) == 0)  # padding rows: zero codes
    _, _, wc, wf = int4_weights(pk, gen)
    assert np.array_equal(host(wf), orc.fp6_chunks(host(wc)))


@pytest.mark.parametrize("m,n,k", [(97, 256, 512), (300, 4096, 1024), (7500, 1024, 4096), (45000, 4096, 1024)])
def test_fp6_gemm_equals_int8_accumulators(pk, m, n, k):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(m + 3 * n + k)
    a = torch.randint(-8, 8, (m, k), generator=gen, device="cuda", dtype=torch.int8)
    b = torch.randint(-8, 8, (n, k), generator=gen, device="cuda", dtype=torch.int8)
    # the FP6 chunk form of the same codes through the library's own encoder:
    # nibble pairs -> pk_unpack_int4_fp6 (checked against the oracle above)
    def fp6_of(c):
        u = (c.to(torch.int16) & 15).to(torch.uint8).view(c.shape[0], -1, 2)
        nib = (u[:, :, 0] | (u[:, :, 1] << 4)).contiguous()
        f = torch.empty(c.shape, dtype=torch.uint8, device="cuda")
        pk.call("pk_unpack_int4_fp6", nib, f, c.numel())
        return f
    af, bf = fp6_of(a), fp6_of(b)
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    note(f"fp6 gemm m={m} n={n} k={k} tile={pk.gemm_tile(pk.FMT_S4F6, pk.EPI_F32, m, n)}")
    pk.gemm(pk.FMT_I8, pk.EPI_I32, a, b, m, n, k, acc)
    pk.gemm(pk.FMT_S4F6, pk.EPI_F32, af, bf, m, n, k, out, in_scale=1.0)
    want = acc.to(torch.float32)
    bad = (out != want).nonzero()
    if bad.numel():
        r, c = bad[0].tolist()
        note(f"fp6 gemm mismatches: {bad.shape[0]} of {m * n}; rows {bad[:, 0].unique().numel()} "
             f"(first {bad[:, 0].min().item()}..{bad[:, 0].max().item()}), cols {bad[:, 1].min().item()}.."
             f"{bad[:, 1].max().item()}; first [{r}, {c}] got {out[r, c].item()} want {want[r, c].item()}; "
             f"nan {torch.isnan(out).sum().item()}")
    assert bad.numel() == 0
    assert acc.abs().max().item() > 0


@pytest.mark.parametrize("t", [272, 1040, 7500, 45000])
def test_fp6_expand_equals_codes(pk, t):
    pad = padded(t) + 16
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2700 + t)
    xc, xcs, xf, xfs = codes_and_fp6(pk, gen, t, pad)
    _, ws, wc, wf = int4_weights(pk, gen)
    c = torch.full((pad * (FF // 2 + FF // 8),), 0x33, dtype=torch.uint8, device="cuda")
    f = torch.full_like(c, 0x44)
    note(f"ffn_expand_int4_sparse_fp6 T={t} tile={pk.gemm_tile(pk.FMT_S4F6, pk.EPI_F8_24, pad, FF)}")
    pk.call("pk_ffn_expand_int4_sparse_codes", xc, wc, ws, xcs, c, pad, 1.0, 1)
    pk.call("pk_ffn_expand_int4_sparse_fp6", xf, wf, ws, xfs, f, pad, 1.0, 1)
    assert torch.equal(c, f)


def test_fp6_producer_nonfinite_rows(pk, orc):
    """Rows holding inf / NaN / huge values take the producer's exact
    (slow) path; their FP6 codes still equal the FP6 form of the int8 codes."""
    t, pad = 96, 112
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2801)
    x = (torch.randn((pad, D), generator=gen, device="cuda") * 2).half()
    x[3, 17] = float("inf")
    x[5, 900] = float("-inf")
    x[8, 5] = float("nan")
    x[11, :] = 65504.0
    x[12, ::2] = -65504.0
    g, b = ln_params(gen)
    xc = torch.full((pad, D), 5, dtype=torch.int8, device="cuda")
    xf = torch.full((pad, D), 0x5A, dtype=torch.uint8, device="cuda")
    s1 = torch.empty(pad, dtype=torch.float32, device="cuda")
    s2 = torch.empty(pad, dtype=torch.float32, device="cuda")
    pk.call("pk_layer_norm_quantize_int4_codes", x, g, b, xc, s1, t, pad, 1e-5)
    pk.call("pk_layer_norm_quantize_int4_fp6", x, g, b, xf, s2, t, pad, 1e-5)
    assert np.array_equal(host(s1).view(np.uint32), host(s2).view(np.uint32))  # NaN scales compare by bits
    codes = host(xc)
    assert codes.min() >= -8 and codes.max() <= 7
    assert np.array_equal(host(xf), orc.fp6_chunks(codes))
