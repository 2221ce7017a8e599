"""Pins of the long-request TDT decode oracle (decoder.cu:452-784,
tdt_persistent_fp8) on the CPU.

- per-tensor INT8 quantization: known answers of the reference's formula
  (scale = max|w| / 127, ties to even, the all-zero matrix);
- one prediction-network update against a float64 restatement from the
  mathematics (dequantized weights x dequantized INT8 states, textbook LSTM
  cell), which fails on a wrong scale, bank, layer, gate order or a dropped
  bias / table term;
- with zero recurrent and layer-1 input weights and one-hot embeddings the
  long form reduces exactly to the fp16 form's decode (pinned separately), so
  the whole loop (state commit, table lookup, projection, joint, frame rules)
  must give the same tokens, final frame and prediction.
"""
import numpy as np
import pytest


def f16(rng, *shape, sc=0.05):
    return (rng.standard_normal(shape) * sc).astype(np.float16)


def test_quantize_tensor_known_answers(oracle):
    w = np.array([127.0, 2.5, 3.5, -2.5, -127.0, 0.49, 126.5, -0.5], np.float16)
    q, s = oracle.quantize_tensor_i8(w)
    assert s == 1.0
    assert q.tolist() == [127, 2, 4, -2, -127, 0, 126, 0]
    z = np.zeros(64, np.float16)
    q, s = oracle.quantize_tensor_i8(z)
    assert s == 1.0 and not q.any()
    # the largest magnitude maps to +-127; the scale is max / 127 in float32
    rng = np.random.default_rng(3)
    w = f16(rng, 4, 64)
    w[2, 5] = -0.3
    q, s = oracle.quantize_tensor_i8(w)
    assert s == np.float32(abs(float(w[2, 5]))) / np.float32(127.0)
    assert q[2, 5] == -127 and np.abs(q).max() == 127
    deq = q.astype(np.float64) * s
    assert np.abs(deq - w.astype(np.float64)).max() <= 0.5 * s * (1 + 1e-6)


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


@pytest.mark.parametrize("with_table", [False, True])
def test_lstm_long_update_against_float64(oracle, with_table):
    H = 128
    rng = np.random.default_rng(11 + with_table)
    w = [f16(rng, 4 * H, H, sc=0.08) for _ in range(3)]  # W_hh0, W_hh1, W_ih1
    qs = [oracle.quantize_tensor_i8(m) for m in w]
    cq = np.array([s / np.float32(127.0) for _, s in qs], np.float32)
    bias = (rng.standard_normal((2, 4 * H)) * 0.2).astype(np.float32)
    table = f16(rng, 4 * H, sc=0.5) if with_table else None
    qh = rng.integers(-127, 128, (2, H)).astype(np.int8)
    c = (rng.standard_normal((2, H)) * 0.5).astype(np.float32)
    qh_out, c_out, h1 = oracle.lstm_long_update(qs[0][0], qs[1][0], qs[2][0], cq, bias, table, qh, c)

    # float64 from the mathematics: W ~ q * scale, h ~ q / 127
    deq = [q.astype(np.float64) * s for q, s in qs]

    def cell(g, cp):
        i, f, gg, o = g[:H], g[H:2 * H], g[2 * H:3 * H], g[3 * H:]
        cn = sigmoid(f) * cp + sigmoid(i) * np.tanh(gg)
        return cn, sigmoid(o) * np.tanh(cn)

    g0 = deq[0] @ (qh[0] / 127.0) + bias[0] + (table.astype(np.float64) if with_table else 0.0)
    c0, h0 = cell(g0, c[0].astype(np.float64))
    q0 = np.clip(np.rint(h0 * 127.0), -127, 127)
    # layer 1's input is the INT8 layer-0 output the oracle produced (a
    # rounding near a tie may legitimately differ from q0 by one step)
    assert np.abs(qh_out[0] - q0).max() <= 1 and (qh_out[0] != q0).mean() < 0.02
    g1 = deq[1] @ (qh[1] / 127.0) + deq[2] @ (qh_out[0] / 127.0) + bias[1]
    c1, h1r = cell(g1, c[1].astype(np.float64))
    np.testing.assert_allclose(c_out[0], c0, atol=2e-6, rtol=0)
    np.testing.assert_allclose(c_out[1], c1, atol=2e-6, rtol=0)
    np.testing.assert_allclose(h1, h1r, atol=2e-6, rtol=0)
    q1 = np.clip(np.rint(h1r * 127.0), -127, 127)
    assert np.abs(qh_out[1] - q1).max() <= 1 and (qh_out[1] != q1).mean() < 0.02


def test_long_decode_reduces_to_fp16_decode(oracle):
    """Zero W_hh0 / W_hh1 / W_ih1 and one-hot embeddings: the long form's
    table rows are exact columns of W_ih0, its recurrent and layer-1 input
    terms vanish, and the decode must equal the fp16 form's."""
    H, T, D, frames = 128, 1025, 5, 64
    rng = np.random.default_rng(77)
    zero = np.zeros((4 * H, H), np.float16)
    w_ih0 = f16(rng, 4 * H, H, sc=0.5)
    # biases on a 2^-8 grid keep b_ih + b_hh + w exact in float32
    b = [(rng.integers(-64, 64, 4 * H) / 256.0).astype(np.float32) for _ in range(4)]
    emb = np.zeros((T - 1, H), np.float16)
    emb[np.arange(T - 1), np.arange(T - 1) % H] = 1.0
    table = np.ascontiguousarray(w_ih0.T[np.arange(T - 1) % H])  # row t = emb[t] x W_ih0^T, exact
    proj = (f16(rng, H, H, sc=0.1), (rng.standard_normal(H) * 0.1).astype(np.float32))
    wj = f16(rng, T + D, H, sc=0.08)
    bj = (rng.standard_normal(T + D) * 0.1).astype(np.float32)
    bj[T - 1] += 1.5
    enc = f16(rng, frames, H, sc=0.5)
    joint = (wj, None, bj)
    lstm16 = (w_ih0, zero, b[0], b[1], zero, zero, b[2], b[3])
    t16, f16_frame, p16 = oracle.tdt_decode(enc, emb, lstm16, proj, joint, T, D)
    tl, fl, pl = oracle.tdt_decode_long(enc, table, (zero, b[0], b[1], zero, zero, b[2], b[3]), proj, joint, T, D)
    assert len(t16) >= 3
    assert np.array_equal(t16, tl) and f16_frame == fl
    np.testing.assert_allclose(pl, p16, atol=1e-6, rtol=0)


def test_deterministic_exp_and_tanh(oracle):
    """The long form's exp / tanh (IEEE basic operations, evaluated the same
    way on the GPU): exp within one ulp of the float64 value over the range
    the cell uses, tanh within 2e-7 absolute, sigmoid limits exact."""
    import math

    lib = oracle.lib()
    xs = np.concatenate([np.linspace(-87.0, 88.0, 40001), np.linspace(-1e-3, 1e-3, 2001), [0.0, -0.0]])
    worst = 0.0
    for x in xs.astype(np.float32):
        e = lib.orc_det_exp(float(x))
        t = math.exp(float(x))
        worst = max(worst, abs(e - t) / float(np.spacing(np.float32(t))))
    assert worst <= 1.0, worst
    assert lib.orc_det_exp(0.0) == 1.0 and lib.orc_det_exp(200.0) == float("inf") and lib.orc_det_exp(-200.0) == 0.0
    for x in np.linspace(-12.0, 12.0, 24001).astype(np.float32):
        assert abs(lib.orc_det_tanh(float(x)) - math.tanh(float(x))) <= 2e-7, x
    assert lib.orc_det_tanh(30.0) == 1.0 and lib.orc_det_tanh(-30.0) == -1.0 and lib.orc_det_tanh(0.0) == 0.0


def test_long_decode_abi_rejects_missing_table_and_bad_shapes():
    """pk_tdt_decode_long validates before any GPU call: a missing input table
    is an argument error (-4), a hidden size off the 128 grid a shape error
    (-1), misaligned recurrent weights an alignment error (-2)."""
    import ctypes
    import os

    lib_path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "l4-parakeet-rs_amd", "build",
                            "libpk_linear.so")
    if not os.path.exists(lib_path):
        pytest.fail("libpk_linear.so is not built")
    lib = ctypes.CDLL(lib_path)
    P, I = ctypes.c_void_p, ctypes.c_int32
    fn = lib.pk_tdt_decode_long
    fn.restype = I
    fn.argtypes = [P, I, I, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I, I, P, I, P, P, ctypes.c_uint64, P]
    buf = ctypes.create_string_buffer(1 << 16)
    base = (ctypes.addressof(buf) + 255) & ~255
    a = P(base)
    ws = lib.pk_tdt_decode_workspace_bytes(640)

    def call(table=a, hidden=640, w=a):
        return fn(a, 16, hidden, table, w, a, a, a, a, a, a, a, a, a, 0, None, a, hidden, 1025, 5, 10, a, 16, a, a, ws,
                  None)

    assert call(table=None) == -4
    assert call(hidden=600) == -1
    assert call(w=P(base + 8)) == -2
