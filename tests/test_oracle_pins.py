"""Pin the CPU oracle before trusting it as the parity checker.

Each test checks one oracle function against something other than its own
formula: the reference's known answers (tests/golden/reference_known_answers.json),
an independent library (numpy float16, torch float8_e4m3fn, numpy int64
matmul, torch SiLU / layer_norm), or a mathematical invariant (round-trip
bounds, exhaustive brute force on small alphabets).
"""
import itertools
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")


@pytest.fixture(scope="module")
def known():
    with open(GOLDEN) as f:
        return json.load(f)


# ---- fp16 ----------------------------------------------------------------------

def test_f16_encode_matches_numpy_rne(oracle):
    rng = np.random.default_rng(1)
    # log-uniform magnitudes across normal, subnormal, overflow and tie points
    mags = np.exp2(rng.uniform(-30, 17, 200000)).astype(np.float32)
    signs = np.where(rng.random(mags.size) < 0.5, -1, 1).astype(np.float32)
    vals = mags * signs
    # exact ties between adjacent halves (RNE must pick the even one)
    h = np.arange(0, 0x7c00, 7, dtype=np.uint16).view(np.float16).astype(np.float32)
    ties = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    vals = np.concatenate([vals, ties, -ties, [0.0, -0.0, 65504.0, 65520.0, 65519.996, 1e-8]]).astype(np.float32)
    ours = oracle.f32_to_f16_bits(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f16_decode_exhaustive(oracle):
    f = oracle.lib().orc_f16_to_f32
    bits = np.arange(0, 0x10000, dtype=np.uint32)
    finite = [b for b in bits if (b & 0x7c00) != 0x7c00]
    ours = np.array([f(int(b)) for b in finite], dtype=np.float32)
    ref = np.array(finite, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


# ---- e4m3 ----------------------------------------------------------------------

def test_e4m3_known_answers(oracle, known):
    for value, code in known["e4m3_encode"]["cases"]:
        assert int(oracle.f32_to_e4m3([value])[0]) == code


def test_e4m3_decode_table_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    table = oracle.e4m3_table()
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(codes)
    assert np.array_equal(np.isnan(table), nan)
    assert np.array_equal(table[~nan], codes[~nan])


def test_e4m3_encode_matches_torch_in_range(oracle):
    torch = pytest.importorskip("torch")
    table = oracle.e4m3_table()
    finite = np.sort(np.unique(np.abs(table[~np.isnan(table)])))
    mids = (finite[:-1] + finite[1:]) / 2  # exact ties -> round to even
    rng = np.random.default_rng(2)
    rand = rng.uniform(-448, 448, 50000).astype(np.float32)
    small = (rng.standard_normal(50000) * 0.01).astype(np.float32)
    vals = np.concatenate([finite, -finite, mids, -mids, rand, small]).astype(np.float32)
    ours = oracle.f32_to_e4m3(vals)
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_saturates(oracle):
    big = np.array([448.0, 449.0, 463.9, 464.0, 500.0, 1e6, np.inf], np.float32)
    assert np.all(oracle.f32_to_e4m3(big) == 0x7E)
    assert np.all(oracle.f32_to_e4m3(-big) == 0xFE)


# ---- int8 / pattern ---------------------------------------------------------------

def test_int8_known_answers(oracle, known):
    for value, q in known["int8_quantize"]["cases"]:
        assert oracle.quantize_i8(value) == q


def test_pattern_spans_both_signs(oracle, known):
    case = known["pattern_both_signs"]
    v = oracle.pattern_fill(case["count"], case["salt"], case["amplitude"])
    assert (v < 0).any() and (v > 0).any()
    assert np.all(np.abs(v) <= case["amplitude"])


# ---- size contracts ----------------------------------------------------------------

def test_estimate_linear_known_answers(oracle, known):
    for case in known["estimate_linear"]["cases"]:
        got = oracle.estimate_linear(case["format"], case["in"], case["out"])
        if case.get("none"):
            assert got is None
            continue
        if "total_bytes" in case:
            assert got["payload_bytes"] + got["metadata_bytes"] == case["total_bytes"]
        for key in ("payload_bytes", "metadata_bytes", "padded_in", "padded_out"):
            if key in case:
                assert got[key] == case[key], (case, got)


def test_exl3_known_answers(oracle, known):
    for case in known["exl3_layout"]["cases"]:
        got = oracle.exl3_layout(case["in"], case["out"], case["bits"])
        for key in ("trellis_shape", "trellis_bytes", "scale_bytes", "padded_in", "padded_out"):
            if key in case:
                assert got[key] == case[key]
    with pytest.raises(ValueError):
        oracle.exl3_layout(0, 4, 4)
    with pytest.raises(ValueError):
        oracle.exl3_layout(4, 4, 9)


def test_pad_fp16_linear_known_answer(oracle, known):
    case = known["pad_fp16_linear"]
    got = oracle.pad_fp16_linear(np.array(case["src"], np.float32), case["padded_out"], case["padded_in"])
    assert got.astype(np.float32).ravel().tolist() == case["expected"]


# ---- packers: round-trip invariants ---------------------------------------------------

def _weights(n, k, seed, sigma=0.02):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, k)) * sigma).astype(np.float16)


def test_pack_int8_rows_round_trip(oracle):
    w = _weights(64, 256, 3)
    q, s = oracle.pack_int8_rows(w)
    wf = w.astype(np.float32)
    assert np.all(np.abs(q.astype(np.float32) * s[:, None] - wf) <= s[:, None] * 0.5 + 1e-9)
    assert np.all(np.abs(q).max(axis=1) == 127)


def test_pack_fp8_rows_round_trip(oracle):
    w = _weights(64, 256, 4)
    q, s = oracle.pack_fp8_rows(w)
    deq = oracle.e4m3_to_f32(q) * s[:, None]
    wf = w.astype(np.float32)
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 for normals, plus the
    # subnormal step 2^-10 * scale
    assert np.all(np.abs(deq - wf) <= np.abs(wf) * 2.0 ** -4 + s[:, None] * 2.0 ** -10)
    assert np.all((q & 0x7F).max(axis=1) == 0x7E)


def test_pack_int4_rows_round_trip_and_nibble_order(oracle):
    w = _weights(32, 128, 5)
    q, s = oracle.pack_int4_rows(w)
    lo = (q & 15).astype(np.int8)
    hi = (q >> 4).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    levels = np.empty((32, 128), np.int8)
    levels[:, 0::2] = lo  # encoder.rs:405: even column in the low nibble
    levels[:, 1::2] = hi
    wf = w.astype(np.float32)
    assert np.all(np.abs(levels * s[:, None] - wf) <= s[:, None] * 0.5 + 1e-7)
    zero_q, zero_s = oracle.pack_int4_rows(np.zeros((1, 8), np.float16))
    assert zero_s[0] == 0.0 and not zero_q.any()


def test_pack_int4_g128_round_trip(oracle):
    w = _weights(16, 512, 6)
    w[3, :128] = 0  # an all-zero group
    q, s, z = oracle.pack_int4_g128(w)
    assert np.all(z.astype(np.float32) == np.round(z.astype(np.float32)))
    levels = np.stack([(q >> (8 * (i % 4) + 4 * (i // 4))) & 15 for i in range(8)], axis=-1).reshape(16, 512)
    deq = (levels - np.repeat(z.astype(np.float32), 128, axis=1)) * np.repeat(s.astype(np.float32), 128, axis=1)
    err = np.abs(deq - w.astype(np.float32))
    assert np.all(err <= np.repeat(s.astype(np.float32), 128, axis=1) * 0.5 + 1e-6)
    assert np.all(deq[3, :128] == 0)


def test_q4k_reference_block_tests(oracle, known):
    case = known["q4k_block"]
    src = oracle.pattern_fill(256, case["pattern_salt"], case["pattern_amplitude"]).astype(np.float16)
    block = oracle.q4k_encode_block(src)
    assert block.size == case["block_bytes"] and block.any()
    zero = oracle.q4k_encode(np.zeros((1, 256), np.float16))
    assert np.all(oracle.q4k_dequant(zero) == 0.0)


def test_q4k_round_trip_error_bound(oracle):
    w = _weights(8, 512, 7)
    blocks = oracle.q4k_encode(w)
    deq = oracle.q4k_dequant(blocks)
    err = np.abs(deq - w.astype(np.float32))
    # per 32-value group the 4-bit grid spans at most the group's range (plus
    # the 6-bit quantisation of scale and min); a wrong nibble/scale placement
    # produces errors of the order of the range itself
    rng_groups = np.ptp(w.astype(np.float32).reshape(8, -1, 32), axis=2)
    bound = np.repeat(rng_groups, 32, axis=1) / 15 * 0.5 * 1.6 + 2e-3
    assert np.all(err <= bound)


# ---- 2:4 compression -------------------------------------------------------------------

def test_compress_24_brute_force(oracle):
    alphabet = [0x00, 0x80, 0x38, 0xB8, 0x40, 0x7E]  # 0, -0, 1, -1, 2, 448
    quartets = np.array(list(itertools.product(alphabet, repeat=4)), np.uint8)
    data, meta = oracle.compress_24(quartets.reshape(1, -1))
    data = data.reshape(-1, 2)
    meta = meta.reshape(-1)
    for p, quartet in enumerate(quartets):
        order = sorted(range(4), key=lambda i: (-(int(quartet[i]) & 127), i))[:2]
        order.sort()
        nib = (meta[p // 2] >> (4 * (p % 2))) & 15
        assert [nib & 3, (nib >> 2) & 3] == order
        assert data[p].tolist() == [int(quartet[order[0]]), int(quartet[order[1]])]


def test_decompress_inverts_compress_on_sparse_rows(oracle):
    rng = np.random.default_rng(8)
    x = rng.integers(1, 255, (4, 64), dtype=np.uint8)
    for r in range(4):
        for p in range(16):
            drop = rng.choice(4, 2, replace=False)
            x[r, 4 * p + drop] = 0
    data, meta = oracle.compress_24(x)
    assert np.array_equal(oracle.decompress_24(data, meta), x)


def test_compress_24_i8_exact_brute_force(oracle):
    """Every quartet over an int8 alphabet with ties, signs, zeros and -128:
    the kept pair is the two largest |v| (ties to the lower index) in index
    order, the overflow holds exactly the other nonzeros in element order,
    and kept pair + overflow rebuild the quartet."""
    alphabet = [0, 1, -1, 2, -2, 127, -127, -128]
    quartets = np.array(list(itertools.product(alphabet, repeat=4)), np.int8)
    row = quartets.reshape(1, -1)
    data, meta, counts, ovf = oracle.compress_24_i8_exact(row)
    data = data.reshape(-1, 2).view(np.int8)
    meta = meta.reshape(-1)
    expect_ovf = []
    for p, quartet in enumerate(quartets):
        order = sorted(range(4), key=lambda i: (-abs(int(quartet[i])), i))[:2]
        order.sort()
        nib = (meta[p // 2] >> (4 * (p % 2))) & 15
        assert [nib & 3, (nib >> 2) & 3] == order
        assert data[p].tolist() == [int(quartet[order[0]]), int(quartet[order[1]])]
        expect_ovf += [((4 * p + i) << 8) | (int(quartet[i]) & 255) for i in range(4) if i not in order and quartet[i] != 0]
    assert counts[0] == len(expect_ovf) <= row.shape[1] // 2
    assert ovf[0, :counts[0]].tolist() == expect_ovf


def test_compress_24_i8_exact_rebuilds_rows(oracle):
    """decompress(2:4 part) + scattered overflow == the row, on dense rows (two
    overflow entries per full quartet: the k/2 bound), sparse and zero rows."""
    rng = np.random.default_rng(10)
    x = rng.integers(-128, 128, (6, 512), dtype=np.int8)
    x[1, rng.random(512) < 0.9] = 0
    x[2] = 0
    x[3] = rng.integers(1, 128, 512)
    data, meta, counts, ovf = oracle.compress_24_i8_exact(x)
    rebuilt = oracle.decompress_24(data, meta).view(np.int8).copy()
    for r in range(6):
        for e in ovf[r, :counts[r]]:
            assert rebuilt[r, e >> 8] == 0
            rebuilt[r, e >> 8] = np.uint8(e & 255).view(np.int8)
    assert np.array_equal(rebuilt, x)
    assert counts[3] == 256 and counts[2] == 0


def test_residual_24_i8_complements_the_selection(oracle):
    """Every quartet over the same alphabet: the residual metadata names the
    two positions the 2:4 selection does not keep, ascending and distinct; its
    bytes are the row's there; its nonzeros are exactly the overflow entries;
    and (2:4 part) + (residual part) rebuild the row, disjointly."""
    alphabet = [0, 1, -1, 2, -2, 127, -127, -128]
    quartets = np.array(list(itertools.product(alphabet, repeat=4)), np.int8)
    row = quartets.reshape(1, -1)
    data, meta, counts, ovf = oracle.compress_24_i8_exact(row)
    data2, meta2 = oracle.residual_24_i8(row, meta)
    m1, m2, d2 = meta.reshape(-1), meta2.reshape(-1), data2.reshape(-1, 2).view(np.int8)
    residual_entries = []
    for p, quartet in enumerate(quartets):
        kept = [int(m1[p // 2] >> (4 * (p % 2))) & 3, int(m1[p // 2] >> (4 * (p % 2) + 2)) & 3]
        nib = (m2[p // 2] >> (4 * (p % 2))) & 15
        rest = [int(nib & 3), int((nib >> 2) & 3)]
        assert rest == sorted(set(range(4)) - set(kept)), (p, kept, rest)
        assert d2[p].tolist() == [int(quartet[rest[0]]), int(quartet[rest[1]])]
        residual_entries += [((4 * p + i) << 8) | (int(quartet[i]) & 255) for i in rest if quartet[i] != 0]
    assert residual_entries == ovf[0, :counts[0]].tolist()
    a = oracle.decompress_24(data, meta).view(np.int8)
    b = oracle.decompress_24(data2, meta2).view(np.int8)
    assert not np.any((a != 0) & (b != 0))
    assert np.array_equal(a.astype(np.int16) + b.astype(np.int16), row.astype(np.int16))


def test_residual_24_i8_rebuilds_rows(oracle):
    rng = np.random.default_rng(12)
    x = rng.integers(-128, 128, (5, 1024), dtype=np.int8)
    x[1, rng.random(1024) < 0.8] = 0
    x[2] = 0
    data, meta, _, _ = oracle.compress_24_i8_exact(x)
    data2, meta2 = oracle.residual_24_i8(x, meta)
    a = oracle.decompress_24(data, meta).view(np.int8).astype(np.int16)
    b = oracle.decompress_24(data2, meta2).view(np.int8).astype(np.int16)
    assert np.array_equal(a + b, x.astype(np.int16))
    assert not data2[2].any()


# ---- GEMMs against numpy --------------------------------------------------------------

def test_gemm_i8_exact(oracle):
    rng = np.random.default_rng(9)
    x = rng.integers(-127, 128, (33, 256), dtype=np.int8)
    w = rng.integers(-127, 128, (48, 256), dtype=np.int8)
    assert np.array_equal(oracle.gemm_i8(x, w), x.astype(np.int64) @ w.astype(np.int64).T)


def test_gemm_s4_exact(oracle):
    rng = np.random.default_rng(10)
    xs = rng.integers(-8, 8, (17, 128))
    ws = rng.integers(-8, 8, (24, 128))

    def pack(a):
        u = (a & 15).astype(np.uint8)
        return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)

    assert np.array_equal(oracle.gemm_s4(pack(xs), pack(ws)), xs @ ws.T)


def test_gemm_e4m3_matches_float64(oracle):
    rng = np.random.default_rng(11)
    x = rng.integers(0, 256, (20, 512)).astype(np.uint8)
    w = rng.integers(0, 256, (24, 512)).astype(np.uint8)
    x[(x & 0x7F) == 0x7F] = 0
    w[(w & 0x7F) == 0x7F] = 0
    t = oracle.e4m3_table().astype(np.float64)
    ref = t[x] @ t[w].T
    got = oracle.gemm_e4m3(x, w)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-3 * np.abs(ref).max())


def test_gemm_g128_paths_match_numpy(oracle):
    rng = np.random.default_rng(12)
    w = _weights(24, 256, 13)
    q, s, z = oracle.pack_int4_g128(w)
    levels = np.stack([(q >> (8 * (i % 4) + 4 * (i // 4))) & 15 for i in range(8)], axis=-1).reshape(24, 256).astype(np.int64)
    zi = np.repeat(z.astype(np.int64), 128, axis=1)
    x16 = rng.standard_normal((9, 256)).astype(np.float16)
    deq = (levels - zi) * np.repeat(s.astype(np.float64), 128, axis=1)
    ref = x16.astype(np.float64) @ deq.T
    assert np.allclose(oracle.gemm_g128_a16(x16, q, s, z), ref, rtol=1e-4, atol=1e-4)
    x8, xs = oracle.quantize_int8_rows(x16)
    out, gacc = oracle.gemm_g128_a8(x8, xs, q, s, z, want_group_acc=True)
    exact = np.einsum("mgk,ngk->mng", x8.astype(np.int64).reshape(9, 2, 128),
                      (levels - zi).reshape(24, 2, 128))
    assert np.array_equal(gacc, exact)


# ---- epilogues / LN / joint against torch ------------------------------------------------

def test_silu_epilogue_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(14)
    acc = rng.standard_normal((8, 64)).astype(np.float32) * 50
    ws = rng.uniform(0.5, 2, 64).astype(np.float32)
    got = oracle.epilogue(acc, 0, ws, in_scale=0.1).astype(np.float32)
    v = torch.from_numpy(acc * np.float32(0.1) * ws)
    ref = torch.nn.functional.silu(v).half().float().numpy()
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3)) <= 2 ** -10


def test_glu_epilogue_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(15)
    acc = rng.standard_normal((6, 32)).astype(np.float32) * 3
    ws = np.ones(32, np.float32)
    got = oracle.epilogue(acc, 5, ws, in_scale=1.0, valid_rows=4).astype(np.float32)
    ref = torch.nn.functional.glu(torch.from_numpy(acc).half().float(), dim=1).numpy()
    assert np.allclose(got[:4], ref[:4], rtol=2e-3, atol=1e-3)
    assert not got[4:].any()


def test_layer_norm_quantize_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(16)
    x = (rng.standard_normal((5, 1024)) * 3 + 1).astype(np.float16)
    g = rng.uniform(0.5, 1.5, 1024).astype(np.float16)
    b = (rng.standard_normal(1024) * 0.1).astype(np.float16)
    q, s, normalized = oracle.layer_norm_quantize(x, g, b, valid_rows=4)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x).float(), (1024,),
                                         torch.from_numpy(g).float(), torch.from_numpy(b).float(),
                                         1e-5).numpy()
    assert np.allclose(normalized[:4].astype(np.float32), ref[:4], rtol=2e-3, atol=2e-3)
    deq = oracle.e4m3_to_f32(q[:4]) * s[:4, None]
    nf = normalized[:4].astype(np.float32)
    assert np.all(np.abs(deq - nf) <= np.abs(nf) * 2 ** -4 + s[:4, None] * 2 ** -10)
    assert s[4] == 1.0 and not q[4].any()


def test_joint_matches_numpy(oracle):
    rng = np.random.default_rng(17)
    w = (rng.standard_normal((1030, 640)) * 0.05).astype(np.float16)
    bias = rng.standard_normal(1030).astype(np.float32)
    enc = rng.standard_normal(640).astype(np.float16)
    pred = rng.standard_normal(640).astype(np.float32)
    inp = np.maximum(enc.astype(np.float64) + pred.astype(np.float64), 0)
    ref = w.astype(np.float64) @ inp + bias
    got = oracle.joint_scores_f16(w, bias, enc, pred)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-4)
    tok, dur = oracle.joint_decide(got)
    assert tok == int(np.argmax(got[:1025])) and dur == int(np.argmax(got[1025:1030]))
    tie = np.zeros(1030, np.float32)
    tie[[7, 9]] = 5.0
    tie[[1027, 1028]] = 1.0
    assert oracle.joint_decide(tie) == (7, 2)


def _scores(token_outputs, durations, token, dur, margin=1.0):
    s = np.zeros(token_outputs + durations, np.float32)
    s[token] = margin
    s[token_outputs + dur] = margin
    return s


def test_joint_scan_frame_rules(oracle):
    """decoder.cu:773-783 closed forms: blank with duration d advances d frames
    per step; blank with duration 0 advances one frame every max_symbols
    steps; a token stops the scan after its own advance."""
    T, D, F = 11, 5, 17
    blank = T - 1
    for d in range(1, D):
        out = oracle.joint_scan(lambda t: _scores(T, D, blank, d), F, token_outputs=T, durations=D)
        assert out == (F + (-F) % d, 0, -1, -(-F // d))
    out = oracle.joint_scan(lambda t: _scores(T, D, blank, 0), F, token_outputs=T, durations=D,
                            max_symbols=3)
    assert out == (F, 0, -1, 3 * F)
    # token 4 at frame 6 with duration 0: stays on frame 6, one symbol added
    f = lambda t: _scores(T, D, 4, 0) if t == 6 else _scores(T, D, blank, 2)
    assert oracle.joint_scan(f, F, token_outputs=T, durations=D) == (6, 1, 4, 4)
    # resuming at frame 6 with 9 symbols: the tenth symbol forces the advance
    assert oracle.joint_scan(f, F, frame=6, symbols=9, token_outputs=T, durations=D) == (7, 0, 4, 1)
    # ties: lower token id and first duration maximum win
    assert oracle.joint_decide(np.zeros(T + D, np.float32), T, D) == (0, 0)


def test_lstm_step_matches_torch_lstm_cell(oracle):
    """The oracle's LSTM cell (gate order i, f, g, o; decoder.cu:116-129)
    against torch.nn.LSTMCell with the same fp16-valued weights."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(170)
    H = 64
    w_ih = (rng.standard_normal((4 * H, H)) * 0.2).astype(np.float16)
    w_hh = (rng.standard_normal((4 * H, H)) * 0.2).astype(np.float16)
    b_ih, b_hh = rng.standard_normal(4 * H).astype(np.float32), rng.standard_normal(4 * H).astype(np.float32)
    x, h, c = (rng.standard_normal(H).astype(np.float32) for _ in range(3))
    cell = torch.nn.LSTMCell(H, H).double()
    with torch.no_grad():
        cell.weight_ih.copy_(torch.from_numpy(w_ih.astype(np.float64)))
        cell.weight_hh.copy_(torch.from_numpy(w_hh.astype(np.float64)))
        cell.bias_ih.copy_(torch.from_numpy(b_ih.astype(np.float64)))
        cell.bias_hh.copy_(torch.from_numpy(b_hh.astype(np.float64)))
        th, tc = cell(torch.from_numpy(x.astype(np.float64))[None], (torch.from_numpy(h.astype(np.float64))[None],
                                                                      torch.from_numpy(c.astype(np.float64))[None]))
    oh, oc = oracle.lstm_step(w_ih, w_hh, b_ih, b_hh, x, h, c)
    assert np.allclose(oh, th[0].numpy(), atol=2e-6) and np.allclose(oc, tc[0].numpy(), atol=2e-6)
    zh, zc = oracle.lstm_step(w_ih, w_hh, b_ih, b_hh, None, h, c)
    with torch.no_grad():
        th, tc = cell(torch.zeros(1, H, dtype=torch.float64), (torch.from_numpy(h.astype(np.float64))[None],
                                                                torch.from_numpy(c.astype(np.float64))[None]))
    assert np.allclose(zh, th[0].numpy(), atol=2e-6) and np.allclose(zc, tc[0].numpy(), atol=2e-6)


def test_tdt_decode_composition(oracle):
    """The decode loop is the joint scan between tokens with the prediction
    network re-run after each token (decoder.cu:733-783 and 616-688): with
    every joint step forced to blank / duration 1, nothing is emitted and the
    prediction is the projection of the zero-input LSTM from the zero state."""
    rng = np.random.default_rng(171)
    H, T, D, frames = 128, 33, 5, 19
    f16 = lambda *s: (rng.standard_normal(s) * 0.1).astype(np.float16)
    f32 = lambda *s: (rng.standard_normal(s) * 0.1).astype(np.float32)
    lstm = (f16(4 * H, H), f16(4 * H, H), f32(4 * H), f32(4 * H), f16(4 * H, H), f16(4 * H, H), f32(4 * H), f32(4 * H))
    proj = (f16(H, H), f32(H))
    bj = f32(T + D)
    bj[T - 1] = 100.0
    bj[T + 1] = 100.0
    toks, frame, pred = oracle.tdt_decode(f16(frames, H), f16(T, H), lstm, proj, (f16(T + D, H), None, bj), T, D)
    assert len(toks) == 0 and frame == frames
    z = np.zeros(H, np.float32)
    h0, c0 = oracle.lstm_step(lstm[0], lstm[1], lstm[2], lstm[3], None, z, z)
    h1, _ = oracle.lstm_step(lstm[4], lstm[5], lstm[6], lstm[7], h0, z, z)
    ref = proj[0].astype(np.float64) @ h1.astype(np.float64) + proj[1]
    assert np.allclose(pred, ref, atol=1e-5)


def _ln64(x, g, b, eps=1e-5):
    x = np.asarray(x, np.float64)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * np.asarray(g, np.float64) + np.asarray(b, np.float64)


def _f16_ulp(v):
    a = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(a)) - 10)


@pytest.mark.parametrize("inverse_scale", [0.0, 56.0])
def test_layer_norm_pair_matches_float64(oracle, inverse_scale):
    """encoder.cu:128-209: the first output is the float64 LayerNorm of x
    rounded to fp16 (within one fp16 ulp; the fp32 statistics may move a
    rounding boundary), the second the float64 LayerNorm of the *rounded*
    first output with the next layer's parameters; the e4m3 form is
    torch's e4m3 of fp16(second) * 56.  The first output also equals the
    normalized output of the single LayerNorm producer bit for bit, and
    padding rows are zero in both outputs."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((9, 1024)) * 2.5 + 0.7).astype(np.float16)
    g1 = rng.uniform(0.5, 1.5, 1024).astype(np.float16)
    b1 = (rng.standard_normal(1024) * 0.1).astype(np.float16)
    g2 = rng.uniform(0.2, 2.0, 1024).astype(np.float16)
    b2 = (rng.standard_normal(1024) * 0.3).astype(np.float16)
    first, second = oracle.layer_norm_pair(x, g1, b1, g2, b2, 1e-5, inverse_scale, valid_rows=7)
    ref1 = _ln64(x[:7], g1, b1)
    f1 = first[:7].astype(np.float64)
    assert np.all(np.abs(f1 - ref1) <= _f16_ulp(ref1))
    assert np.mean(f1 == ref1.astype(np.float16)) > 0.99
    _, _, normalized = oracle.layer_norm_quantize(x, g1, b1, 1e-5, valid_rows=7)
    assert np.array_equal(first.view(np.uint16), normalized.view(np.uint16))
    ref2 = _ln64(f1, g2, b2)
    sec16 = oracle.layer_norm_pair(x, g1, b1, g2, b2, 1e-5, 0.0, valid_rows=7)[1]
    s2 = sec16[:7].astype(np.float64)
    assert np.all(np.abs(s2 - ref2) <= _f16_ulp(ref2))
    assert np.mean(s2 == ref2.astype(np.float16)) > 0.99
    # the second LayerNorm must not run on x itself
    assert np.max(np.abs(s2 - _ln64(x[:7], g2, b2))) > 1e-2
    if inverse_scale:
        want = torch.from_numpy(np.clip(sec16[:7].astype(np.float32) * np.float32(56.0), -448, 448))
        assert np.array_equal(second[:7], want.to(torch.float8_e4m3fn).view(torch.uint8).numpy())
    else:
        assert np.array_equal(second.view(np.uint16), sec16.view(np.uint16))
    assert not first[7:].view(np.uint16).any() and not np.asarray(second[7:]).view(np.uint8).any()
