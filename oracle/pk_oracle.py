"""numpy front end for the C oracle (oracle/pk_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
Every function forwards to the C restatement, which cites the reference
file:line it follows.  fp16 arrays are numpy float16 (same bits as uint16).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libpk_oracle.so")

_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float
S = ctypes.c_size_t


def _declare(l):
    sig = {
        "orc_f32_to_f16": (ctypes.c_uint16, [F]),
        "orc_f16_to_f32": (F, [ctypes.c_uint16]),
        "orc_f32_to_e4m3": (ctypes.c_uint8, [F]),
        "orc_e4m3_to_f32": (F, [ctypes.c_uint8]),
        "orc_e3m2_to_f32": (F, [ctypes.c_uint8]),
        "orc_e3m2_of_int": (ctypes.c_uint8, [I]),
        "orc_fp6_chunks": (None, [P, S, P]),
        "orc_quantize_i8": (ctypes.c_int8, [F]),
        "orc_pattern": (F, [ctypes.c_uint64, ctypes.c_uint64, F]),
        "orc_pattern_fill": (None, [P, S, ctypes.c_uint64, ctypes.c_uint64, F]),
        "orc_estimate_linear": (I, [I, S, S, I, P]),
        "orc_exl3_layout": (I, [S, S, I, P]),
        "orc_pack_fp8_rows": (None, [P, I, I, P, P]),
        "orc_pack_int8_rows": (None, [P, I, I, P, P]),
        "orc_pack_int4_rows": (None, [P, I, I, P, P]),
        "orc_pack_int4_g128": (None, [P, I, I, P, P, P]),
        "orc_pad_fp16_linear": (None, [P, I, I, I, I, P]),
        "orc_q4k_encode_block": (None, [P, P]),
        "orc_q4k_value": (F, [P, I]),
        "orc_q4k_encode": (None, [P, I, I, P]),
        "orc_quantize_fp8_static": (None, [P, S, F, P]),
        "orc_quantize_int8_static": (None, [P, S, F, P]),
        "orc_quantize_fp8_rows": (None, [P, I, I, I, P, P]),
        "orc_quantize_int8_rows": (None, [P, I, I, I, P, P]),
        "orc_quantize_int4_rows": (None, [P, I, I, I, P, P]),
        "orc_layer_norm_quantize": (None, [P, P, P, I, I, I, F, I, P, P, P]),
        "orc_layer_norm_pair": (None, [P, P, P, P, P, I, I, F, F, P, P]),
        "orc_compress_24_i8_exact": (None, [P, I, I, P, P, P, P]),
        "orc_residual_24_i8": (None, [P, P, I, I, P, P]),
        "orc_compress_24": (None, [P, I, I, P, P]),
        "orc_decompress_24": (None, [P, P, I, I, P]),
        "orc_gemm_i8_i32": (None, [P, P, I, I, I, P]),
        "orc_gemm_s4_i32": (None, [P, P, I, I, I, P]),
        "orc_gemm_e4m3_f32": (None, [P, P, I, I, I, P]),
        "orc_gemm_f16_f32": (None, [P, P, I, I, I, P]),
        "orc_gemm_g128_a16": (None, [P, P, P, P, I, I, I, P]),
        "orc_gemm_g128_a8": (None, [P, P, P, P, P, I, I, I, I, P, P]),
        "orc_gemm_q4k_f32": (None, [P, P, I, I, I, P]),
        "orc_gemm_g128_f8": (None, [P, P, P, P, I, I, I, P]),
        "orc_epilogue": (None, [P, P, F, P, P, I, I, I, I, P, P]),
        "orc_epilogue_linear": (None, [P, P, P, I, I, F, F, I, P]),
        "orc_epilogue_quantized": (None, [P, F, P, P, I, I, I, P]),
        "orc_joint_scores_f16": (None, [P, P, P, P, I, I, P]),
        "orc_joint_scores_i8": (None, [P, P, P, P, P, I, I, P]),
        "orc_joint_decide": (None, [P, I, I, P, P]),
        "orc_lstm_step": (None, [P, P, P, P, P, P, P, I, P, P]),
        "orc_tdt_decode": (I, [P, I, I, P, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I, I, P, I, P, P]),
        "orc_det_exp": (F, [F]),
        "orc_det_tanh": (F, [F]),
        "orc_quantize_tensor_i8": (F, [P, S, P]),
        "orc_lstm_long_update": (None, [P, P, P, P, P, P, P, P, I, P, P, P]),
        "orc_tdt_decode_long": (I, [P, I, I, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I, I, P, I, P, P]),
        "orc_score_vector_byte": (I, [I]),
        "orc_key_int4_nibble": (I, [I]),
        "orc_pack_score_vectors": (None, [P, I, P, P]),
        "orc_pack_key_int4": (None, [P, I, P, P]),
        "orc_quantize_value_int4": (None, [P, I, F, I, I, P]),
        "orc_local_attention": (None, [I, P, P, P, P, P, P, P, I, I, I, I, I, I, P, P, P, P, I, I]),
        "orc_quantize_fp8_transpose": (None, [P, I, F, P]),
        "orc_pack_position_heads": (None, [P, P]),
        "orc_local_attention_short": (None, [P, P, P, P, P, P, P, I, I, I, I, I]),
        "orc_threads": (I, []),
        "orc_set_threads": (None, [I]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _h(a):
    """Return a C-contiguous float16 view as the C side's uint16."""
    a = np.ascontiguousarray(a)
    assert a.dtype in (np.float16, np.uint16)
    return a


# ---- scalars ---------------------------------------------------------------

def f32_to_e4m3(values) -> np.ndarray:
    v = np.asarray(values, dtype=np.float32).ravel()
    f = lib().orc_f32_to_e4m3
    return np.array([f(float(x)) for x in v], dtype=np.uint8)


def e4m3_table() -> np.ndarray:
    f = lib().orc_e4m3_to_f32
    return np.array([f(i) for i in range(256)], dtype=np.float32)


def e4m3_to_f32(codes) -> np.ndarray:
    return e4m3_table()[np.asarray(codes, dtype=np.uint8)]


def e3m2_to_f32(bits: int) -> float:
    return lib().orc_e3m2_to_f32(int(bits))


def e3m2_of_int(v: int) -> int:
    return lib().orc_e3m2_of_int(int(v))


def fp6_chunks(codes: np.ndarray) -> np.ndarray:
    """int8 codes (any shape, size a multiple of 16) -> the FP6 e3m2 chunk form
    as uint8 of the same shape (orc_fp6_chunks)."""
    c = np.ascontiguousarray(codes, dtype=np.int8)
    out = np.empty(c.shape, dtype=np.uint8)
    lib().orc_fp6_chunks(_p(c), c.size, _p(out))
    return out


def f32_to_f16_bits(values) -> np.ndarray:
    v = np.asarray(values, dtype=np.float32).ravel()
    f = lib().orc_f32_to_f16
    return np.array([f(float(x)) for x in v], dtype=np.uint16)


def quantize_i8(value: float) -> int:
    return int(lib().orc_quantize_i8(float(value)))


def pattern(index: int, salt: int, amplitude: float) -> float:
    return float(lib().orc_pattern(index, salt, amplitude))


def pattern_fill(count: int, salt: int, amplitude: float, first: int = 0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().orc_pattern_fill(_p(out), count, first, salt, amplitude)
    return out


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


# ---- size contracts ----------------------------------------------------------

FORMATS = {"fp16": 0, "fp8_e4m3": 1, "int8": 2, "q4_k": 3, "exl3": 4}


def estimate_linear(fmt: str, logical_in: int, logical_out: int, exl3_bits: int = 4):
    out = np.zeros(6, dtype=np.uint64)
    status = lib().orc_estimate_linear(FORMATS[fmt], logical_in, logical_out, exl3_bits, _p(out))
    if status < 0:
        raise ValueError(f"estimate_linear error {status}")
    if status == 0:
        return None
    keys = ("logical_in", "logical_out", "padded_in", "padded_out", "payload_bytes",
            "metadata_bytes")
    return {k: int(v) for k, v in zip(keys, out)}


def exl3_layout(logical_in: int, logical_out: int, qbits: int):
    out = np.zeros(7, dtype=np.uint64)
    status = lib().orc_exl3_layout(logical_in, logical_out, qbits, _p(out))
    if status != 0:
        raise ValueError(f"exl3 error {status}")
    o = [int(v) for v in out]
    return {"padded_in": o[0], "padded_out": o[1], "trellis_shape": o[2:5],
            "trellis_bytes": o[5], "scale_bytes": o[6]}


# ---- packers -------------------------------------------------------------------

def pack_fp8_rows(w16: np.ndarray):
    w16 = _h(w16)
    n, k = w16.shape
    q = np.empty((n, k), np.uint8)
    s = np.empty(n, np.float32)
    lib().orc_pack_fp8_rows(_p(w16), n, k, _p(q), _p(s))
    return q, s


def pack_int8_rows(w16: np.ndarray):
    w16 = _h(w16)
    n, k = w16.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().orc_pack_int8_rows(_p(w16), n, k, _p(q), _p(s))
    return q, s


def pack_int4_rows(w16: np.ndarray):
    w16 = _h(w16)
    n, k = w16.shape
    q = np.empty((n, k // 2), np.uint8)
    s = np.empty(n, np.float32)
    lib().orc_pack_int4_rows(_p(w16), n, k, _p(q), _p(s))
    return q, s


def pack_int4_g128(w16: np.ndarray):
    w16 = _h(w16)
    n, k = w16.shape
    q = np.empty((n, k // 8), np.uint32)
    s = np.empty((n, k // 128), np.float16)
    z = np.empty((n, k // 128), np.float16)
    lib().orc_pack_int4_g128(_p(w16), n, k, _p(q), _p(s), _p(z))
    return q, s, z


def pad_fp16_linear(src: np.ndarray, padded_out: int, padded_in: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32)
    lo, li = src.shape
    dst = np.empty((padded_out, padded_in), np.float16)
    lib().orc_pad_fp16_linear(_p(src), lo, li, padded_out, padded_in, _p(dst))
    return dst


def q4k_encode(w16: np.ndarray) -> np.ndarray:
    w16 = _h(w16)
    n, k = w16.shape
    out = np.empty((n, k // 256, 144), np.uint8)
    lib().orc_q4k_encode(_p(w16), n, k, _p(out))
    return out


def q4k_encode_block(src256: np.ndarray) -> np.ndarray:
    src = _h(np.asarray(src256, dtype=np.float16))
    out = np.empty(144, np.uint8)
    lib().orc_q4k_encode_block(_p(src), _p(out))
    return out


def q4k_dequant(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n, per_row, _ = blocks.shape
    out = np.empty((n, per_row * 256), np.float32)
    f = lib().orc_q4k_value
    for r in range(n):
        for b in range(per_row):
            ptr = blocks[r, b].ctypes.data
            for i in range(256):
                out[r, b * 256 + i] = f(ptr, i)
    return out


# ---- activation quantizers ---------------------------------------------------

def quantize_fp8_static(x16: np.ndarray, inverse_scale: float) -> np.ndarray:
    x16 = _h(x16)
    out = np.empty(x16.shape, np.uint8)
    lib().orc_quantize_fp8_static(_p(x16), x16.size, inverse_scale, _p(out))
    return out


def quantize_int8_static(x16: np.ndarray, inverse_scale: float) -> np.ndarray:
    x16 = _h(x16)
    out = np.empty(x16.shape, np.int8)
    lib().orc_quantize_int8_static(_p(x16), x16.size, inverse_scale, _p(out))
    return out


def quantize_fp8_rows(x16: np.ndarray, valid_rows: int | None = None):
    x16 = _h(x16)
    m, k = x16.shape
    q = np.empty((m, k), np.uint8)
    s = np.empty(m, np.float32)
    lib().orc_quantize_fp8_rows(_p(x16), m, m if valid_rows is None else valid_rows, k,
                                _p(q), _p(s))
    return q, s


def quantize_int8_rows(x16: np.ndarray, valid_rows: int | None = None):
    x16 = _h(x16)
    m, k = x16.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    lib().orc_quantize_int8_rows(_p(x16), m, m if valid_rows is None else valid_rows, k,
                                 _p(q), _p(s))
    return q, s


def quantize_int4_rows(x16: np.ndarray, valid_rows: int | None = None):
    x16 = _h(x16)
    m, k = x16.shape
    q = np.empty((m, k // 2), np.uint8)
    s = np.empty(m, np.float32)
    lib().orc_quantize_int4_rows(_p(x16), m, m if valid_rows is None else valid_rows, k,
                                 _p(q), _p(s))
    return q, s


def layer_norm_quantize(x16, gamma16, beta16, epsilon=1e-5, int4=False, valid_rows=None):
    x16 = _h(x16)
    m, k = x16.shape
    assert k == 1024
    q = np.empty((m, k // 2 if int4 else k), np.uint8)
    s = np.empty(m, np.float32)
    normalized = np.empty((m, k), np.float16)
    lib().orc_layer_norm_quantize(_p(x16), _p(_h(gamma16)), _p(_h(beta16)), m,
                                  m if valid_rows is None else valid_rows, k, epsilon,
                                  1 if int4 else 0, _p(q), _p(s), _p(normalized))
    return q, s, normalized


def layer_norm_pair(x16, w1, b1, w2, b2, epsilon=1e-5, inverse_scale=0.0, valid_rows=None):
    """LayerNorm pair (encoder.cu:128-209): returns (first fp16 [m x 1024],
    second as fp16 [m x 1024] or e4m3 bytes when inverse_scale != 0)."""
    x16 = _h(x16)
    m, k = x16.shape
    assert k == 1024
    out = np.empty((m, k), np.float16)
    nxt = np.empty((m, k), np.uint8 if inverse_scale != 0.0 else np.float16)
    lib().orc_layer_norm_pair(_p(x16), _p(_h(w1)), _p(_h(b1)), _p(_h(w2)), _p(_h(b2)), m,
                              m if valid_rows is None else valid_rows, epsilon, inverse_scale,
                              _p(out), _p(nxt))
    return out, nxt


def compress_24(x8: np.ndarray):
    x8 = np.ascontiguousarray(x8, dtype=np.uint8)
    m, k = x8.shape
    data = np.empty((m, k // 2), np.uint8)
    meta = np.empty((m, k // 8), np.uint8)
    lib().orc_compress_24(_p(x8), m, k, _p(data), _p(meta))
    return data, meta


def compress_24_i8_exact(x8: np.ndarray):
    """INT8 rows -> (2:4 data, metadata, overflow counts, overflow lists);
    entry j of row r is (element << 8) | byte, lists padded with zeros to k/2."""
    x8 = np.ascontiguousarray(x8, dtype=np.int8)
    m, k = x8.shape
    data = np.empty((m, k // 2), np.uint8)
    meta = np.empty((m, k // 8), np.uint8)
    counts = np.empty(m, np.uint32)
    ovf = np.zeros((m, k // 2), np.uint32)
    lib().orc_compress_24_i8_exact(_p(x8), m, k, _p(data), _p(meta), _p(counts), _p(ovf))
    return data, meta, counts, ovf


def residual_24_i8(x8: np.ndarray, meta: np.ndarray):
    """INT8 rows and their 2:4 metadata -> (residual data, residual metadata):
    per quartet the two positions the metadata does not keep, ascending."""
    x8 = np.ascontiguousarray(x8, dtype=np.int8)
    meta = np.ascontiguousarray(meta, dtype=np.uint8)
    m, k = x8.shape
    data2 = np.empty((m, k // 2), np.uint8)
    meta2 = np.empty((m, k // 8), np.uint8)
    lib().orc_residual_24_i8(_p(x8), _p(meta), m, k, _p(data2), _p(meta2))
    return data2, meta2


def decompress_24(data: np.ndarray, meta: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    meta = np.ascontiguousarray(meta, dtype=np.uint8)
    m, half = data.shape
    out = np.empty((m, half * 2), np.uint8)
    lib().orc_decompress_24(_p(data), _p(meta), m, half * 2, _p(out))
    return out


# ---- GEMMs --------------------------------------------------------------------

def gemm_i8(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    m, k = x.shape
    n = w.shape[0]
    acc = np.empty((m, n), np.int32)
    lib().orc_gemm_i8_i32(_p(x), _p(w), m, n, k, _p(acc))
    return acc


def gemm_s4(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint8)
    w = np.ascontiguousarray(w, np.uint8)
    m, kh = x.shape
    n = w.shape[0]
    acc = np.empty((m, n), np.int32)
    lib().orc_gemm_s4_i32(_p(x), _p(w), m, n, kh * 2, _p(acc))
    return acc


def gemm_e4m3(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint8)
    w = np.ascontiguousarray(w, np.uint8)
    m, k = x.shape
    n = w.shape[0]
    acc = np.empty((m, n), np.float32)
    lib().orc_gemm_e4m3_f32(_p(x), _p(w), m, n, k, _p(acc))
    return acc


def gemm_f16(x16: np.ndarray, w16: np.ndarray) -> np.ndarray:
    x16 = _h(x16)
    w16 = _h(w16)
    m, k = x16.shape
    n = w16.shape[0]
    acc = np.empty((m, n), np.float32)
    lib().orc_gemm_f16_f32(_p(x16), _p(w16), m, n, k, _p(acc))
    return acc


def gemm_g128_a16(x16, q, s, z) -> np.ndarray:
    x16 = _h(x16)
    m, k = x16.shape
    n = q.shape[0]
    out = np.empty((m, n), np.float32)
    lib().orc_gemm_g128_a16(_p(x16), _p(np.ascontiguousarray(q)), _p(_h(s)), _p(_h(z)),
                            m, n, k, _p(out))
    return out


def gemm_g128_a8(x8, x_scales, q, s, z, want_group_acc=False, parts=1):
    x8 = np.ascontiguousarray(x8, np.int8)
    m, k = x8.shape
    n = q.shape[0]
    out = np.empty((m, n), np.float32)
    gacc = np.empty((m, n, k // 128), np.int32) if want_group_acc else None
    lib().orc_gemm_g128_a8(_p(x8), _p(np.ascontiguousarray(x_scales, np.float32)),
                           _p(np.ascontiguousarray(q)), _p(_h(s)), _p(_h(z)), m, n, k, parts,
                           _p(gacc), _p(out))
    return (out, gacc) if want_group_acc else out


def gemm_g128_f8(x8, q, s, z) -> np.ndarray:
    """e4m3 activations [m x k] x INT4-g128 weights: the fp32 accumulator
    before the epilogue (group sums rounded once, folded with one fma each)."""
    x8 = np.ascontiguousarray(x8, np.uint8)
    m, k = x8.shape
    n = q.shape[0]
    out = np.empty((m, n), np.float32)
    lib().orc_gemm_g128_f8(_p(x8), _p(np.ascontiguousarray(q, np.uint32)), _p(_h(s)), _p(_h(z)), m, n, k, _p(out))
    return out


def gemm_q4k(x16, blocks) -> np.ndarray:
    x16 = _h(x16)
    m, k = x16.shape
    n = blocks.shape[0]
    acc = np.empty((m, n), np.float32)
    lib().orc_gemm_q4k_f32(_p(x16), _p(np.ascontiguousarray(blocks, np.uint8)), m, n, k,
                           _p(acc))
    return acc


# ---- epilogues ----------------------------------------------------------------

def epilogue(acc, mode, w_scales, row_scales=None, in_scale=1.0, bias=None, residual=None,
             valid_rows=None):
    """ffn_fp8_async epilogue restatement; returns fp16 or e4m3 array."""
    acc = np.ascontiguousarray(acc, np.float32)
    m, n = acc.shape
    ws = np.ascontiguousarray(w_scales, np.float32)
    rs = None if row_scales is None else np.ascontiguousarray(row_scales, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    out8 = None
    if mode == 5:
        out16 = np.zeros((m, n // 2), np.float16)
    elif mode in (2, 6, 8):
        out16 = np.array(residual, dtype=np.float16, copy=True, order="C")
    else:
        out16 = np.zeros((m, n), np.float16)
    if mode in (1, 7, 9):
        out8 = np.zeros((m, n), np.uint8)
    lib().orc_epilogue(_p(acc), _p(rs), in_scale, _p(ws), _p(b), m, n, mode,
                       m if valid_rows is None else valid_rows, _p(out16), _p(out8))
    return out8 if mode in (1, 7, 9) else out16


def epilogue_linear(acc, bias=None, residual=None, out_scale=1.0, res_scale=0.0,
                    activation=0) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.float32)
    m, n = acc.shape
    out = np.empty((m, n), np.float16)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    r = None if residual is None else _h(residual)
    lib().orc_epilogue_linear(_p(acc), _p(b), _p(r), m, n, out_scale, res_scale, activation,
                              _p(out))
    return out


def epilogue_quantized(acc, in_scale, w_scales, bias=None, activation=0) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.float32)
    m, n = acc.shape
    out = np.empty((m, n), np.float16)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_epilogue_quantized(_p(acc), in_scale, _p(np.ascontiguousarray(w_scales, np.float32)),
                                 _p(b), m, n, activation, _p(out))
    return out


# ---- joint --------------------------------------------------------------------

def joint_scores_f16(w16, bias, enc16, pred):
    w16 = _h(w16)
    o, h = w16.shape
    out = np.empty(o, np.float32)
    lib().orc_joint_scores_f16(_p(w16), _p(np.ascontiguousarray(bias, np.float32)), _p(_h(enc16)),
                               _p(np.ascontiguousarray(pred, np.float32)), o, h, _p(out))
    return out


def joint_scores_i8(wq, w_scales, bias, enc16, pred):
    wq = np.ascontiguousarray(wq, np.int8)
    o, h = wq.shape
    out = np.empty(o, np.float32)
    lib().orc_joint_scores_i8(_p(wq), _p(np.ascontiguousarray(w_scales, np.float32)),
                              _p(np.ascontiguousarray(bias, np.float32)), _p(_h(enc16)),
                              _p(np.ascontiguousarray(pred, np.float32)), o, h, _p(out))
    return out


def joint_decide(scores, token_outputs=1025, durations=5):
    scores = np.ascontiguousarray(scores, np.float32)
    tok = ctypes.c_int()
    dur = ctypes.c_int()
    lib().orc_joint_decide(_p(scores), token_outputs, durations, ctypes.byref(tok),
                           ctypes.byref(dur))
    return tok.value, dur.value


def joint_scan(scores_of_frame, frames, frame=0, symbols=0, token_outputs=1025, durations=5,
               max_symbols=10):
    """decoder.cu:733-783 with the prediction vector fixed: greedy TDT joint
    steps from (frame, symbols) until a non-blank token (id token_outputs-1 is
    the blank) or the frames run out.  scores_of_frame(t) returns the fp32
    scores of frame t.  Returns (frame, symbols, token or -1, steps)."""
    blank = token_outputs - 1
    steps = 0
    while frame < frames:
        tok, dur = joint_decide(scores_of_frame(frame), token_outputs, durations)
        steps += 1
        symbols += 1
        frame += dur
        if dur != 0 or symbols == max_symbols:
            if dur == 0:
                frame += 1
            symbols = 0
        if tok != blank:
            return frame, symbols, tok, steps
    return frame, symbols, -1, steps


def lstm_step(w_ih, w_hh, b_ih, b_hh, x, h, c):
    """decoder.cu:116-129: one LSTM layer step; x None = zero input."""
    w_ih, w_hh = _h(w_ih), _h(w_hh)
    hidden = w_ih.shape[1]
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    ho = np.empty(hidden, np.float32)
    co = np.empty(hidden, np.float32)
    lib().orc_lstm_step(_p(w_ih), _p(w_hh), _p(f32(b_ih)), _p(f32(b_hh)), None if x is None else _p(f32(x)),
                        _p(f32(h)), _p(f32(c)), hidden, _p(ho), _p(co))
    return ho, co


def tdt_decode(enc, emb, lstm, proj, joint, token_outputs=1025, durations=5, max_symbols=10, capacity=None):
    """decoder.cu:146-445 greedy TDT decode.  lstm = (w_ih0, w_hh0, b_ih0, b_hh0,
    w_ih1, w_hh1, b_ih1, b_hh1) (fp16 weights [4H x H], fp32 biases); proj =
    (w fp16 [H x H], b fp32 [H]); joint = (w fp16 or int8 [O x H], scales or
    None, b fp32 [O]).  Returns (tokens, final frame, final prediction)."""
    enc = _h(enc)
    frames, hidden = enc.shape
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    w_ih0, w_hh0, b_ih0, b_hh0, w_ih1, w_hh1, b_ih1, b_hh1 = lstm
    wj, sj, bj = joint
    int8 = np.asarray(wj).dtype == np.int8
    wj = np.ascontiguousarray(wj)
    capacity = capacity or frames * max_symbols
    toks = np.empty(capacity, np.int32)
    pred = np.empty(hidden, np.float32)
    frame = ctypes.c_int()
    keep = [f32(b_ih0), f32(b_hh0), f32(b_ih1), f32(b_hh1), f32(proj[1]), f32(bj),
            None if sj is None else f32(sj)]
    n = lib().orc_tdt_decode(_p(enc), frames, hidden, _p(_h(emb)), _p(_h(w_ih0)), _p(_h(w_hh0)), _p(keep[0]),
                             _p(keep[1]), _p(_h(w_ih1)), _p(_h(w_hh1)), _p(keep[2]), _p(keep[3]),
                             _p(_h(proj[0])), _p(keep[4]), _p(wj), int(int8), _p(keep[6]) if int8 else None,
                             _p(keep[5]), hidden, token_outputs, durations, max_symbols, _p(toks), capacity,
                             _p(pred), ctypes.byref(frame))
    return toks[:min(n, capacity)].copy(), frame.value, pred


def quantize_tensor_i8(w):
    """decoder.cu:520-575 per-tensor symmetric INT8 -> (int8 array, scale)."""
    w = _h(w)
    q = np.empty(w.shape, np.int8)
    return q, float(lib().orc_quantize_tensor_i8(_p(w), w.size, _p(q)))


def lstm_long_update(q_hh0, q_hh1, q_ih1, cq, bias, table_row, qh, c):
    """decoder.cu:613-672: one long-form prediction-network update.  bias =
    [2 x 4H] (b_ih + b_hh per layer), qh int8 [2 x H], c float32 [2 x H];
    table_row fp16 [4H] or None.  Returns (qh', c', h1')."""
    hidden = qh.shape[-1]
    qh_out = np.empty((2, hidden), np.int8)
    c_out = np.empty((2, hidden), np.float32)
    h1 = np.empty(hidden, np.float32)
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    cq, bias, c = f32(cq), f32(bias), f32(c)
    i8 = lambda a: np.ascontiguousarray(a, np.int8)
    q_hh0, q_hh1, q_ih1, qh = i8(q_hh0), i8(q_hh1), i8(q_ih1), i8(qh)
    lib().orc_lstm_long_update(_p(q_hh0), _p(q_hh1), _p(q_ih1), _p(cq), _p(bias),
                               None if table_row is None else _p(_h(table_row)), _p(qh), _p(c), hidden, _p(qh_out),
                               _p(c_out), _p(h1))
    return qh_out, c_out, h1


def tdt_decode_long(enc, table, lstm, proj, joint, token_outputs=1025, durations=5, max_symbols=10, capacity=None):
    """decoder.cu:452-784 greedy TDT decode with the long-request prediction
    network.  table = fp16 [(token_outputs - 1) x 4H] layer-0 input terms;
    lstm = (w_hh0, b_ih0, b_hh0, w_ih1, w_hh1, b_ih1, b_hh1); proj and joint as
    tdt_decode.  Returns (tokens, final frame, final prediction)."""
    enc = _h(enc)
    frames, hidden = enc.shape
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    w_hh0, b_ih0, b_hh0, w_ih1, w_hh1, b_ih1, b_hh1 = lstm
    wj, sj, bj = joint
    int8 = np.asarray(wj).dtype == np.int8
    wj = np.ascontiguousarray(wj)
    capacity = capacity or frames * max_symbols
    toks = np.empty(capacity, np.int32)
    pred = np.empty(hidden, np.float32)
    frame = ctypes.c_int()
    keep = [f32(b_ih0), f32(b_hh0), f32(b_ih1), f32(b_hh1), f32(proj[1]), f32(bj),
            None if sj is None else f32(sj)]
    n = lib().orc_tdt_decode_long(_p(enc), frames, hidden, _p(_h(table)), _p(_h(w_hh0)), _p(keep[0]), _p(keep[1]),
                                  _p(_h(w_ih1)), _p(_h(w_hh1)), _p(keep[2]), _p(keep[3]), _p(_h(proj[0])),
                                  _p(keep[4]), _p(wj), int(int8), _p(keep[6]) if int8 else None, _p(keep[5]), hidden,
                                  token_outputs, durations, max_symbols, _p(toks), capacity, _p(pred),
                                  ctypes.byref(frame))
    return toks[:min(n, capacity)].copy(), frame.value, pred


# ---- local relative-position attention (encoder.cu:1476-2097) -----------------

MODEL_WIDTH, HEAD_WIDTH, HEADS, POSITION_ROWS = 1024, 128, 8, 272


def pack_score_vectors(x16: np.ndarray):
    """encoder.cu:2054-2074: INT8 per-128-vector packing in MMA byte order."""
    x16 = _h(x16)
    vectors = x16.size // 128
    out = np.empty(vectors * 128, np.uint8)
    sc = np.empty(vectors, np.float32)
    lib().orc_pack_score_vectors(_p(x16), vectors, _p(out), _p(sc))
    return out, sc


def pack_key_int4(x16: np.ndarray):
    """encoder.cu:2076-2097: INT4 per-128-vector packing, 64 bytes per vector."""
    x16 = _h(x16)
    vectors = x16.size // 128
    out = np.empty(vectors * 64, np.uint8)
    sc = np.empty(vectors, np.float32)
    lib().orc_pack_key_int4(_p(x16), vectors, _p(out), _p(sc))
    return out, sc


def quantize_value_int4(vt16: np.ndarray, inverse_scale: float = 56.0, edge_only: bool = False,
                        valid_rows: int | None = None, fill: int = 0) -> np.ndarray:
    """encoder.cu:561-634: feature-major V [1024 x rows] -> FP8 V, S4 V, scales.
    Bytes the edge-only form does not write keep the value `fill`."""
    vt16 = _h(vt16)
    rows = vt16.shape[1]
    elements = rows * MODEL_WIDTH
    out = np.full(elements + elements // 2 + 4 * MODEL_WIDTH, fill, np.uint8)
    lib().orc_quantize_value_int4(_p(vt16), rows, inverse_scale, int(edge_only),
                                  rows if valid_rows is None else valid_rows, _p(out))
    return out


def local_attention(packed, query, key, value_fp8, position, bias_u, bias_v, rows, valid_rows=None,
                    value_stride=None, packed_key=None, key_scales=None, packed_position=None,
                    position_scales=None, tiles=None, left=128, right=128, out=None):
    """encoder.cu:1476-2052 long-form local attention over query tiles `tiles`
    (range of 16-row tiles; default all).  Returns the output [padded_rows x
    1024]: e4m3 bytes when packed, fp16 bits otherwise."""
    query, key, position = _h(query), _h(key), _h(position)
    padded_rows = query.shape[0]
    valid_rows = rows if valid_rows is None else valid_rows
    value_stride = padded_rows if value_stride is None else value_stride
    if out is None:
        out = np.zeros((padded_rows, MODEL_WIDTH), np.uint8 if packed else np.uint16)
    t0, t1 = (0, (padded_rows + 15) // 16) if tiles is None else tiles
    f32 = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
    ks, ps = f32(key_scales), f32(position_scales)
    lib().orc_local_attention(int(bool(packed)), _p(query), _p(key), _p(np.ascontiguousarray(value_fp8)),
                              _p(position), _p(_h(bias_u)), _p(_h(bias_v)), _p(out), rows, padded_rows, valid_rows,
                              left, right, value_stride, _p(packed_key), _p(ks), _p(packed_position), _p(ps), t0, t1)
    return out


def quantize_fp8_transpose(x16: np.ndarray, inverse_scale: float) -> np.ndarray:
    """encoder.cu:644-671: row-major fp16 [rows x 1024] -> e4m3 [1024 x rows]."""
    x16 = _h(x16)
    rows = x16.shape[0]
    out = np.empty((MODEL_WIDTH, rows), np.uint8)
    lib().orc_quantize_fp8_transpose(_p(x16), rows, inverse_scale, _p(out))
    return out


def pack_position_heads(x16: np.ndarray) -> np.ndarray:
    """encoder.cu:1321-1336: [272 x 1024] -> [8 x 272 x 128] fp16."""
    x16 = _h(x16)
    out = np.empty((HEADS, POSITION_ROWS, HEAD_WIDTH), np.float16)
    lib().orc_pack_position_heads(_p(x16), _p(out))
    return out


def local_attention_short(query, key, value, position, bias_u, bias_v, rows, valid_rows=None, left=128, right=128):
    """encoder.cu:1338-1461 short-form attention; position = packed [8 x 272 x
    128].  Returns fp16 [padded_rows x 1024]."""
    query, key, value, position = _h(query), _h(key), _h(value), _h(position)
    padded_rows = query.shape[0]
    valid_rows = rows if valid_rows is None else valid_rows
    out = np.empty((padded_rows, MODEL_WIDTH), np.float16)
    lib().orc_local_attention_short(_p(query), _p(key), _p(value), _p(position), _p(_h(bias_u)), _p(_h(bias_v)),
                                    _p(out), rows, padded_rows, valid_rows, left, right)
    return out

