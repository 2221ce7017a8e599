"""Exact 2:4 activation-sparse FF2 against the oracle.

The producer (pk_quantize_rows_int8_sparse24) must give the INT8 bytes and
scales of the dense per-row quantizer, the reference's 2:4 selection of them
(encoder.cu:685-704) and the overflow lists of the dropped nonzeros, bit for
bit.  The contract (pk_ffn_contract_int8_sparse24) must give the dense INT8
contract's fp32 output bit for bit: compared in full with the row-skip
kernel on the dense rows and on sampled rows with the oracle's integer
matmul.  Cases: the config's per-frame top-k sparsity sweep at T = 7500,
dense rows (two overflow entries in most quartets, several overflow chunks
per tile), zero and padding rows, a row with inf, ragged row counts.
"""
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
    print(f"[gpu-sparse24] {msg}", flush=True)
    sys.stdout.flush()


def host(t):
    torch.cuda.synchronize()
    a = t.cpu()
    if a.dtype == torch.float16:
        return a.view(torch.int16).numpy().view(np.float16)
    return a.numpy()


def topk_silu(t, k, sparsity, gen):
    """SiLU(N(0,1)) fp16 rows keeping each frame's top (1 - sparsity) magnitudes."""
    a = torch.nn.functional.silu(torch.randn((t, k), generator=gen, device="cuda")).half()
    keep = max(1, int(round(k * (1.0 - sparsity))))
    thr = a.abs().float().kthvalue(k - keep + 1, dim=1, keepdim=True).values
    return torch.where(a.abs().float() >= thr, a, torch.zeros_like(a))


def produce(pk, x, valid_rows=None, residual=False):
    t, k = x.shape
    data = torch.empty((t, k // 2), dtype=torch.uint8, device="cuda")
    meta = torch.empty((t, k // 8), dtype=torch.uint8, device="cuda")
    scales = torch.empty(t, dtype=torch.float32, device="cuda")
    counts = torch.empty(t, dtype=torch.int32, device="cuda")
    ovf = torch.zeros((t, k // 2), dtype=torch.int32, device="cuda")
    data2 = torch.full((t, k // 2), 0x5A, dtype=torch.uint8, device="cuda") if residual else None
    meta2 = torch.full((t, k // 8), 0x5A, dtype=torch.uint8, device="cuda") if residual else None
    pk.call("pk_quantize_rows_int8_sparse24", x, data, meta, scales, counts, ovf, data2, meta2, t,
            t if valid_rows is None else valid_rows, k)
    return data, meta, scales, counts, ovf, data2, meta2


def check_producer(pk, orc, x, valid_rows=None, rows=None, residual=False):
    data, meta, scales, counts, ovf, data2, meta2 = produce(pk, x, valid_rows, residual)
    xh = host(x)
    q, s = orc.quantize_int8_rows(xh, valid_rows)
    rd, rm, rc, ro = orc.compress_24_i8_exact(q)
    idx = np.arange(x.shape[0]) if rows is None else rows
    assert np.array_equal(host(scales)[idx], s[idx]), "scales"
    assert np.array_equal(host(data)[idx], rd[idx]), "2:4 data"
    assert np.array_equal(host(meta)[idx], rm[idx]), "metadata"
    c = host(counts).view(np.uint32)
    assert np.array_equal(c[idx], rc[idx]), "overflow counts"
    o = host(ovf).view(np.uint32)
    for r in idx:
        assert np.array_equal(o[r, :c[r]], ro[r, :rc[r]]), f"overflow list of row {r}"
    if residual:
        r2d, r2m = orc.residual_24_i8(q, rm)
        assert np.array_equal(host(data2)[idx], r2d[idx]), "residual data"
        assert np.array_equal(host(meta2)[idx], r2m[idx]), "residual metadata"
    return q, s


@pytest.mark.parametrize("k", [1024, 1152, 4096])
def test_producer_exact_edge_rows(pk, orc, k):
    """Random dense rows, zero rows, a row with inf, all-equal magnitudes
    (ties), padding rows past valid_rows; k = 1152 leaves lanes idle in the
    last chunk round (partial wave ballots)."""
    note(f"sparse24 producer edge rows k={k}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(k)
    t = 40
    x = torch.randn((t, k), generator=gen, device="cuda").half()
    x[3] = 0
    x[5, 7] = float("inf")
    x[6] = 0.5
    x[7, ::2] = -0.5
    x[7, 1::2] = 0.5
    x[8] = topk_silu(1, k, 0.9, gen)[0]
    check_producer(pk, orc, x, valid_rows=36, residual=True)
    check_producer(pk, orc, x, valid_rows=36)


@pytest.mark.parametrize("sparsity", [0.5, 0.8, 0.9, 0.95])
def test_producer_exact_T7500(pk, orc, sparsity):
    note(f"sparse24 producer T=7500 sparsity={sparsity}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(int(sparsity * 1000))
    x = topk_silu(7500, 4096, sparsity, gen)
    rows = np.unique(np.concatenate([np.arange(0, 7500, 97), [7499]]))
    check_producer(pk, orc, x, rows=rows, residual=True)


def test_transpose_int8(pk):
    note("transpose int8 1030 x 4096")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    w = torch.randint(-128, 128, (1030, 4096), generator=gen, device="cuda", dtype=torch.int32).to(torch.int8)
    wt = torch.empty((4096, 1030), dtype=torch.int8, device="cuda")
    pk.call("pk_transpose_int8", w, wt, 1030, 4096)
    assert np.array_equal(host(wt), host(w).T)


def int8_weights(pk, gen, n=1024, k=4096):
    w16 = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).half()
    wq = torch.empty((n, k), dtype=torch.int8, device="cuda")
    ws = torch.empty(n, dtype=torch.float32, device="cuda")
    pk.call("pk_pack_int8_rows", w16, n, k, wq, ws)
    wt = torch.empty((k, n), dtype=torch.int8, device="cuda")
    pk.call("pk_transpose_int8", wq, wt, n, k)
    return wq, wt, ws


def run_contract(pk, orc, x, gen, sample, residual):
    t, k = x.shape
    wq, wt, ws = int8_weights(pk, gen)
    data, meta, scales, counts, ovf, data2, meta2 = produce(pk, x, residual=residual)
    out = torch.empty((t, 1024), dtype=torch.float32, device="cuda")
    pk.call("pk_ffn_contract_int8_sparse24", data, meta, scales, counts, ovf, data2, meta2, wq, wt, ws, out, t)
    # dense INT8 rows of the same quantizer, through the dense row-skip contract
    xq = torch.empty((t, k), dtype=torch.int8, device="cuda")
    xs = torch.empty(t, dtype=torch.float32, device="cuda")
    pk.call("pk_quantize_rows", 1, x, xq, xs, t, t, k)
    dense = torch.empty((t, 1024), dtype=torch.float32, device="cuda")
    pk.call("pk_ffn_contract_int8_rowskip", xq, xs, wq, ws, dense, t, None)
    got = host(out)
    assert np.array_equal(got, host(dense)), "sparse24 output differs from the dense INT8 contract"
    acc = orc.gemm_i8(host(xq)[sample], host(wq)).astype(np.float32)
    ref = (acc * host(xs)[sample][:, None]).astype(np.float32) * host(ws)[None, :]
    assert np.array_equal(got[sample], ref.astype(np.float32)), "sparse24 output differs from the oracle"
    return int(host(counts).sum())


@pytest.mark.parametrize("residual", [False, True])
@pytest.mark.parametrize("sparsity", [0.5, 0.8, 0.9, 0.95])
def test_contract_exact_T7500(pk, orc, sparsity, residual):
    """With the residual form, the 50 % and 80 % tiles (385 / 30 overflow
    entries per row) take the second sparse pass, the 90 % and 95 % tiles
    (4 / 0.5) the lists."""
    note(f"sparse24 contract T=7500 sparsity={sparsity} residual={residual}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7 + int(sparsity * 100))
    x = topk_silu(7500, 4096, sparsity, gen)
    sample = np.unique(np.concatenate([np.arange(0, 7500, 128) + (np.arange(59) * 37) % 128, [7499]]))
    sample = sample[sample < 7500]
    entries = run_contract(pk, orc, x, gen, sample, residual)
    note(f"  overflow entries per row {entries / 7500:.2f}")


@pytest.mark.parametrize("residual", [False, True])
@pytest.mark.parametrize("t", [1, 5, 129, 300])
def test_contract_exact_dense_and_ragged(pk, orc, t, residual):
    """Dense random rows (about two overflow entries per quartet: hundreds of
    thousands per 128-row tile, so many overflow chunks), zero rows, ragged
    row counts."""
    note(f"sparse24 contract dense/ragged t={t} residual={residual}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(100 + t)
    x = torch.randn((t, 4096), generator=gen, device="cuda").half()
    if t > 3:
        x[2] = 0
        x[3] = topk_silu(1, 4096, 0.95, gen)[0]
    run_contract(pk, orc, x, gen, np.arange(t), residual)
