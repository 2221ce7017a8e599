"""Full-size parity: the GEMM kernel variants the benchmark times, at the
BASELINE sizes, against the CPU oracle on sampled rows.

The launcher picks the tile height from the grid (pk_gemm_tile reports it),
so small test shapes never reach the 256-row kernels that run the T = 7500 /
45000 linears.  Every case here asserts the tile it runs, then compares a
sample of output rows -- at least one row of every 256-row strip, the first
and the ragged last row -- over all N columns with the oracle applied to the
same quantized rows (the reference's own check of timed outputs samples rows
the same way, quant_benchmark.rs:832-909).  INT8 and INT4-g128 x INT8 results
are compared bit for bit (fp16 / fp32 outputs whose epilogue has no
transcendental); FP8 and fp16-activation results within max|err| <= 1e-2 *
RMS of the output (residual outputs: of residual + update, the stated form,
and the update alone within 2e-2 of its own RMS); e4m3 outputs of the SiLU epilogue within one e4m3 step on < 1 % of codes
(the device exp differs from the host's by <= 1 ulp).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 1e-2
D, FF, CONV = 1024, 4096, 2048
# (name, n_out, k_in, epilogue kind) of one FastConformer layer's linears
LINEARS = [
    ("ff1_expand", FF, D, "f8"),
    ("ff1_contract", D, FF, "res_half"),
    ("qkv", 3 * D, D, "f16"),
    ("attn_out", D, D, "res"),
    ("pw1", CONV, D, "f16"),
    ("pw2", D, D, "res"),
    ("ff2_expand", FF, D, "f8"),
    ("ff2_contract", D, FF, "res_half"),
]


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
    print(f"[gpu-fullsize] {msg}", flush=True)
    sys.stdout.flush()


def sample_rows(m, seed, per_strip=1):
    """At least `per_strip` rows of every 256-row strip (offsets varying by
    strip so that every row position inside a tile is reached somewhere),
    plus the first and the last row."""
    rng = np.random.default_rng(seed)
    rows = {0, m - 1}
    for s in range(0, m, 256):
        for off in rng.integers(0, 256, per_strip):
            rows.add(min(m - 1, s + int(off)))
    return np.array(sorted(rows), np.int64)


def rows_of(t, idx):
    """Host copy of rows `idx` of a device tensor (fp16 as numpy float16)."""
    torch.cuda.synchronize()
    sel = t[torch.from_numpy(idx).cuda()]
    a = sel.cpu()
    if a.dtype == torch.float16:
        return a.view(torch.int16).numpy().view(np.float16)
    if a.dtype == torch.int8:
        return a.numpy()
    return a.numpy()


def host(t):
    torch.cuda.synchronize()
    a = t.cpu()
    if a.dtype == torch.float16:
        return a.view(torch.int16).numpy().view(np.float16)
    return a.numpy()


def assert_close(got, ref, tol=TOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    err = np.max(np.abs(got - ref))
    assert np.isfinite(got).all(), what
    assert err <= tol * rms, f"{what}: max err {err} > {tol} * rms {rms}"


def assert_fp8_close(table, got, ref, exact_frac=0.99, what=""):
    same = np.mean(got == ref)
    assert same >= exact_frac, f"{what}: only {same:.4f} of e4m3 codes equal"
    g, r = table[got].astype(np.float64), table[ref].astype(np.float64)
    assert np.all(np.abs(g - r) <= np.abs(r) / 8 + 2.0 ** -9 + 1e-12), what


def pack(pk, fmt, n, k, gen):
    w16 = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).half()
    if fmt == "fp8":
        q = torch.empty((n, k), dtype=torch.uint8, device="cuda")
        s = torch.empty(n, dtype=torch.float32, device="cuda")
        pk.call("pk_pack_fp8_rows", w16, n, k, q, s)
        return q, s, None
    if fmt == "int8":
        q = torch.empty((n, k), dtype=torch.int8, device="cuda")
        s = torch.empty(n, dtype=torch.float32, device="cuda")
        pk.call("pk_pack_int8_rows", w16, n, k, q, s)
        return q, s, None
    q = torch.empty((n, k // 8), dtype=torch.int32, device="cuda")
    s = torch.empty((n, k // 128), dtype=torch.float16, device="cuda")
    z = torch.empty((n, k // 128), dtype=torch.float16, device="cuda")
    pk.call("pk_pack_int4_g128", w16, n, k, q, s, z)
    return q, s, z


def activations(pk, t, k, kind, gen, outliers=True):
    """fp16 ~N(0,1) with 0.1 % outliers at +-20, quantized
    per row on the GPU (kind 0 FP8, 1 INT8); the quantizer is pinned bit-exact
    elsewhere, and only its output is used here."""
    x = torch.randn((t, k), generator=gen, device="cuda")
    if outliers:
        m = torch.rand((t, k), generator=gen, device="cuda") < 1e-3
        sign = torch.where(torch.rand((t, k), generator=gen, device="cuda") < 0.5, -20.0, 20.0)
        x = torch.where(m, sign, x)
    x = x.half()
    q = torch.empty((t, k), dtype=torch.uint8 if kind == 0 else torch.int8, device="cuda")
    sc = torch.empty(t, dtype=torch.float32, device="cuda")
    pk.call("pk_quantize_rows", kind, x, q, sc, t, t, k)
    return q, sc


class Layer:
    """One layer's eight linears in one format at T frames, run through
    pk_gemm exactly as the benchmark's stack runs them."""

    def __init__(self, pk, orc, fmt, t, seed):
        self.pk, self.orc, self.fmt, self.t = pk, orc, fmt, t
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        kind = 0 if fmt == "fp8" else 1
        self.x4, self.s4 = activations(pk, t, FF, kind, gen)
        self.x1, self.s1 = activations(pk, t, D, kind, gen)
        self.state = torch.randn((t, D), generator=gen, device="cuda").half()
        self.gen = gen
        self.rows = sample_rows(t, seed)
        self.table = orc.e4m3_table()

    def host_acc(self, xq, xs, q, s, z):
        """Oracle result of the sampled rows before the epilogue, with the row
        scale already applied for INT4-g128 (whose oracle folds it in), and the
        matching weight scales."""
        orc = self.orc
        if self.fmt == "fp8":
            return orc.gemm_e4m3(xq, host(q)), xs, host(s)
        if self.fmt == "int8":
            return orc.gemm_i8(xq, host(q)).astype(np.float32), xs, host(s)
        out = orc.gemm_g128_a8(xq, xs, host(q).view(np.uint32), host(s), host(z))
        return out, None, np.ones(q.shape[0], np.float32)

    def check(self, name, n, k, epi):
        pk, orc, t = self.pk, self.orc, self.t
        f = {"fp8": pk.FMT_FP8, "int8": pk.FMT_I8, "int4g128": pk.FMT_G128A8}[self.fmt]
        q, s, z = pack(pk, self.fmt, n, k, self.gen)
        a, xs = (self.x4, self.s4) if k == FF else (self.x1, self.s1)
        ws = None if self.fmt == "int4g128" else s
        gs, gz = (s, z) if self.fmt == "int4g128" else (None, None)
        e = pk.EPI_F8 if epi == "f8" else pk.EPI_F16
        rows_tile, _ = pk.gemm_tile(f, e, t, n)
        note(f"{self.fmt} {name} T={t} n={n} k={k} epi={epi} tile_rows={rows_tile} sampled={len(self.rows)}")
        idx = self.rows
        xq = rows_of(a, idx)
        xsh = rows_of(xs, idx)
        acc, rs, wsh = self.host_acc(xq, xsh, q, s, z)
        exact = self.fmt != "fp8"
        what = f"{self.fmt} {name} T={t}"
        if epi == "f8":
            out = torch.empty((t, n), dtype=torch.uint8, device="cuda")
            pk.gemm(f, pk.EPI_F8, a, q, t, n, k, out, w_scales=ws, row_scales=xs, g_scales=gs, g_zeros=gz)
            ref = orc.epilogue(acc, 1, wsh, row_scales=rs)
            assert_fp8_close(self.table, rows_of(out, idx), ref, 0.99, what)
        elif epi == "f16":
            out = torch.empty((t, n), dtype=torch.float16, device="cuda")
            pk.gemm(f, pk.EPI_F16, a, q, t, n, k, out, w_scales=ws, row_scales=xs, g_scales=gs, g_zeros=gz)
            ref = orc.epilogue(acc, 3, wsh, row_scales=rs, bias=np.zeros(n, np.float32))
            got = rows_of(out, idx)
            if exact:
                assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), what
            else:
                assert_close(got, ref, what=what)
        else:
            half = epi == "res_half"
            before = rows_of(self.state, idx)
            pk.gemm(f, pk.EPI_F16, a, q, t, n, k, self.state, w_scales=ws, row_scales=xs, residual=self.state,
                    out_scale=0.5 if half else 1.0, res_scale=1.0, g_scales=gs, g_zeros=gz)
            ref = orc.epilogue(acc, 2 if half else 6, wsh, row_scales=rs, residual=before)
            got = rows_of(self.state, idx)
            if exact:
                assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), what
            else:
                assert_close(got, ref, what=what + " (output)")
                d_ref = ref.astype(np.float32) - before.astype(np.float32)
                d_got = got.astype(np.float32) - before.astype(np.float32)
                assert_close(d_got, d_ref, tol=2e-2, what=what + " (update)")
        return rows_tile


# ---- one FP8 layer at T = 7500 ----------------------------------

def test_c2_fp8_layer_T7500(pk, orc):
    """QKV (fp16), attention out (+residual), FF1 (e4m3 SiLU), FF2 (+0.5
    residual), conv pointwise 1 (fp16), all FP8 weights and per-row FP8
    activations at T = 7500: the 256-row kernels for N = 2048 and 4096,
    128-row kernels for N = 1024 and for QKV (720 tiles of 256 rows would
    leave the second round of 512 workgroups 40 % full)."""
    layer = Layer(pk, orc, "fp8", 7500, 0x5EED0002)
    want = {"qkv": 128, "attn_out": 128, "ff1_expand": 256, "ff2_contract": 128, "pw1": 256}
    for name, n, k, epi in LINEARS:
        if name in want:
            assert layer.check(name, n, k, epi) == want[name], name


# ---- one stack layer at T = 45000 in each format ----------------

@pytest.mark.parametrize("fmt", ["fp8", "int8", "int4g128"])
def test_stack_layer_T45000(pk, orc, fmt):
    """All eight linears of a stack layer at T = 45000 with the benchmark's
    epilogues: every one runs a 256-row kernel (<fmt, e4m3 SiLU | fp16 |
    fp16 + residual, 256 rows>)."""
    layer = Layer(pk, orc, fmt, 45000, 0x5EED0005 + len(fmt))
    for name, n, k, epi in LINEARS:
        assert layer.check(name, n, k, epi) == 256, name
    del layer
    torch.cuda.empty_cache()


# ---- INT4-g128 FF1 / FF2 at T = 7500 and 45000 --------------------

@pytest.mark.parametrize("t", [7500, 45000])
def test_c3_int4g128_full(pk, orc, t):
    """INT4-g128 weights (fp16 scales / zero-points) with fp16 activations
    (within 1e-2 RMS) and with per-token INT8 activations (fp32 output bit
    for bit, i.e. exact INT8 group accumulators), FF1 1024 -> 4096 and FF2
    4096 -> 1024."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5EED0003 + t)
    idx = sample_rows(t, t)
    for name, n, k in (("ff1", FF, D), ("ff2", D, FF)):
        q, s, z = pack(pk, "int4g128", n, k, gen)
        qh, sh, zh = host(q).view(np.uint32), host(s), host(z)
        x = torch.randn((t, k), generator=gen, device="cuda").half()
        out = torch.empty((t, n), dtype=torch.float32, device="cuda")
        note(f"g128 a16 {name} T={t} tile={pk.gemm_tile(pk.FMT_G128A16, pk.EPI_F32, t, n)}")
        pk.call("pk_linear_int4g128", x, q, s, z, None, out, 1, t, n, k)
        assert_close(rows_of(out, idx), orc.gemm_g128_a16(rows_of(x, idx), qh, sh, zh), what=f"a16 {name} T={t}")
        xq = torch.empty((t, k), dtype=torch.int8, device="cuda")
        xs = torch.empty(t, dtype=torch.float32, device="cuda")
        pk.call("pk_quantize_rows", 1, x, xq, xs, t, t, k)
        note(f"g128 a8 {name} T={t} tile={pk.gemm_tile(pk.FMT_G128A8, pk.EPI_F32, t, n)}")
        pk.call("pk_linear_int4g128_a8", xq, xs, q, s, z, None, out, 1, t, n, k)
        ref = orc.gemm_g128_a8(rows_of(xq, idx), rows_of(xs, idx), qh, sh, zh)
        assert np.array_equal(rows_of(out, idx), ref), f"a8 {name} T={t}"
        del x, xq, out
    torch.cuda.empty_cache()


# ---- activation-sparse FF2 at T = 7500 ----------------------------

@pytest.mark.parametrize("sparsity", [0.5, 0.8, 0.9, 0.95])
def test_c4_rowskip_T7500(pk, orc, sparsity):
    """INT8 row-skip FF2 (4096 -> 1024, fp32 out) on SiLU-like activations
    keeping each frame's top (1 - sparsity) magnitudes, plus 640 padding
    frames of zeros (whose all-zero 16 x 128 blocks the kernel skips):
    exact fp32 outputs on sampled rows, and the skip counters count the
    padding blocks."""
    t, n, k, pad = 7500, 1024, 4096, 640
    gen = torch.Generator(device="cuda")
    gen.manual_seed(int(sparsity * 100))
    a = torch.nn.functional.silu(torch.randn((t, k), generator=gen, device="cuda")).half()
    keep = max(1, int(round(k * (1.0 - sparsity))))
    thr = a.abs().float().kthvalue(k - keep + 1, dim=1, keepdim=True).values
    a = torch.where(a.abs().float() >= thr, a, torch.zeros_like(a))
    a[t - pad:] = 0
    xq = torch.empty((t, k), dtype=torch.int8, device="cuda")
    xs = torch.empty(t, dtype=torch.float32, device="cuda")
    pk.call("pk_quantize_rows", 1, a, xq, xs, t, t, k)
    wq, ws, _ = pack(pk, "int8", n, k, gen)
    out = torch.empty((t, n), dtype=torch.float32, device="cuda")
    counts = torch.zeros(2, dtype=torch.int32, device="cuda")
    note(f"rowskip sparsity={sparsity} tile={pk.gemm_tile(pk.FMT_I8_SKIP, pk.EPI_F32, t, n)}")
    assert pk.gemm_tile(pk.FMT_I8_SKIP, pk.EPI_F32, t, n)[0] == 128
    pk.call("pk_ffn_contract_int8_rowskip", xq, xs, wq, ws, out, t, counts)
    idx = np.union1d(sample_rows(t, 77), np.array([t - pad - 1, t - pad, t - 1]))
    acc = orc.gemm_i8(rows_of(xq, idx), host(wq)).astype(np.float32)
    ref = (acc * rows_of(xs, idx)[:, None]).astype(np.float32) * host(ws)[None, :]
    assert np.array_equal(rows_of(out, idx), ref.astype(np.float32))
    skipped, total = (int(v) for v in host(counts))
    # Each wave counts its 16-row blocks per K-step, and the two waves of a
    # row half share its rows: 2 x (16-row blocks of the 128-row tiles) x
    # column tiles x K-steps.  Every block from the first whole block of
    # padding frames on (rows past t read row t - 1, also zero) is skipped.
    row_blocks = (t + 127) // 128 * 8
    steps, col_tiles = k // 128, n // 128
    assert total == 2 * row_blocks * col_tiles * steps, total
    zero_blocks = row_blocks - (t - pad + 15) // 16
    assert skipped >= 2 * zero_blocks * col_tiles * steps, (skipped, total)


# ---- activation producers at the stack's size --------------------------------------
# One wave per row with rows strided over a grid of at most 8 blocks per CU, so
# at T = 45000 every wave works through several rows (the small parity tests
# give each wave at most one).  Sampled rows, padding rows included, against
# the oracle bit for bit.

@pytest.mark.parametrize("int4", [False, True])
def test_layer_norm_quantize_T45000(pk, orc, int4):
    t, pad = 45000, 45056
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4500 + int(int4))
    x = (torch.randn((pad, D), generator=gen, device="cuda") * 2 + 0.3).half()
    g = (torch.rand(D, generator=gen, device="cuda") + 0.5).half()
    b = (torch.randn(D, generator=gen, device="cuda") * 0.1).half()
    out = torch.empty((pad, D // 2 if int4 else D), dtype=torch.uint8, device="cuda")
    scales = torch.empty(pad, dtype=torch.float32, device="cuda")
    name = "pk_layer_norm_quantize_int4_dynamic" if int4 else "pk_layer_norm_quantize_fp8_dynamic"
    note(f"layer_norm_quantize T={t} padded={pad} int4={int4}")
    pk.call(name, x, g, b, out, scales, t, pad, 1e-5)
    idx = np.union1d(sample_rows(pad, 31 + int(int4), per_strip=2), np.arange(t - 3, pad))
    q, s, _ = orc.layer_norm_quantize(rows_of(x, idx), host(g), host(b), 1e-5, int4, valid_rows=int((idx < t).sum()))
    assert np.array_equal(host(scales)[idx], s)
    assert np.array_equal(rows_of(out, idx), q)


@pytest.mark.parametrize("kind,k", [(0, D), (1, FF), (2, D)])
def test_quantize_rows_T45000(pk, orc, kind, k):
    t, valid = 45000, 44990
    gen = torch.Generator(device="cuda")
    gen.manual_seed(450 + kind)
    x = torch.randn((t, k), generator=gen, device="cuda").half()
    out = torch.empty((t, k // 2 if kind == 2 else k), dtype=torch.uint8, device="cuda")
    scales = torch.empty(t, dtype=torch.float32, device="cuda")
    note(f"quantize_rows T={t} k={k} kind={kind}")
    pk.call("pk_quantize_rows", kind, x, out, scales, t, valid, k)
    idx = np.union1d(sample_rows(t, 41 + kind, per_strip=2), np.arange(valid - 3, t))
    ref = {0: orc.quantize_fp8_rows, 1: orc.quantize_int8_rows, 2: orc.quantize_int4_rows}[kind](
        rows_of(x, idx), int((idx < valid).sum()))
    assert np.array_equal(host(scales)[idx], ref[1])
    assert np.array_equal(rows_of(out, idx).view(np.uint8), ref[0].view(np.uint8))


@pytest.mark.parametrize("m,n,k", [(7500, 1024, 4096), (45000, 4096, 1024), (2000, 3072, 1024)])
def test_fp32_outputs_large_grid(pk, orc, m, n, k):
    """fp32 outputs of the occupancy-2 engine (FP8 / INT8 formats store them
    from the deferred epilogue, 16 bytes per instruction): INT8 at unit scales
    equals its int32 accumulators exactly, FP8 matches the oracle on sampled
    rows within 1e-2 * RMS.  Regression test for a store whose data registers
    were rewritten before the store had read them (rows 12-15 of 16-row
    blocks came out wrong)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(m + n + k)
    a = torch.randint(-127, 128, (m, k), generator=gen, device="cuda", dtype=torch.int8)
    b = torch.randint(-127, 128, (n, k), generator=gen, device="cuda", dtype=torch.int8)
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    note(f"fp32 outputs INT8 m={m} n={n} k={k} tile={pk.gemm_tile(pk.FMT_I8, pk.EPI_F32, m, n)}")
    pk.gemm(pk.FMT_I8, pk.EPI_I32, a, b, m, n, k, acc)
    pk.gemm(pk.FMT_I8, pk.EPI_F32, a, b, m, n, k, out, in_scale=1.0)
    assert torch.equal(out, acc.to(torch.float32))
    x8 = (torch.randn((m, k), generator=gen, device="cuda") * 2).to(torch.float8_e4m3fn).view(torch.uint8)
    w8 = (torch.randn((n, k), generator=gen, device="cuda") * 2).to(torch.float8_e4m3fn).view(torch.uint8)
    out.fill_(float("nan"))
    note(f"fp32 outputs FP8 m={m} n={n} k={k} tile={pk.gemm_tile(pk.FMT_FP8, pk.EPI_F32, m, n)}")
    pk.gemm(pk.FMT_FP8, pk.EPI_F32, x8, w8, m, n, k, out, in_scale=1.0)
    idx = sample_rows(m, m + 7)
    assert_close(rows_of(out, idx), orc.gemm_e4m3(rows_of(x8, idx), host(w8)), what=f"fp8 fp32 out m={m}")
    assert not torch.isnan(out).any()
