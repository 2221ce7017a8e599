"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and its host-only size contracts give the reference's
known answers (no GPU is touched)."""
import ctypes
import json
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pk_linear.h")
LIB = os.path.join(ROOT, "l4-parakeet-rs_amd", "build", "libpk_linear.so")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int32_t|void)\s+(pk_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libpk_linear.so is not built (run __graft_entry__.build())")
    return ctypes.CDLL(LIB)


def test_header_declares_the_boundary():
    syms = declared_symbols()
    assert len(syms) >= 30
    for name in ("pk_linear_fp8_epilogue", "pk_linear_int8_epilogue", "pk_ffn_contract_fp8",
                 "pk_joint_gemv", "pk_pack_int4_g128", "pk_estimate_linear"):
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing


def test_python_mirror_covers_every_symbol():
    import importlib.util

    spec = importlib.util.spec_from_file_location(
        "pk_sig", os.path.join(ROOT, "l4-parakeet-rs_amd", "parakeet_linear", "__init__.py"))
    text = open(spec.origin).read()
    for s in declared_symbols():
        assert f'"{s}"' in text, s


def _estimate(lib, fmt, lin, lout, bits=4):
    fn = lib.pk_estimate_linear
    fn.argtypes = [ctypes.c_int32, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int32, ctypes.c_void_p]
    fn.restype = ctypes.c_int32
    out = np.zeros(6, np.uint64)
    st = fn(fmt, lin, lout, bits, out.ctypes.data)
    return st, out


def test_estimate_linear_matches_reference_tests(lib):
    known = json.load(open(GOLDEN))
    fmts = {"fp16": 0, "fp8_e4m3": 1, "int8": 2, "q4_k": 3, "exl3": 4}
    for case in known["estimate_linear"]["cases"]:
        st, out = _estimate(lib, fmts[case["format"]], case["in"], case["out"])
        if case.get("none"):
            assert st == 0
            continue
        assert st == 1
        if "total_bytes" in case:
            assert int(out[4] + out[5]) == case["total_bytes"]
        for key, idx in (("payload_bytes", 4), ("metadata_bytes", 5), ("padded_in", 2), ("padded_out", 3)):
            if key in case:
                assert int(out[idx]) == case[key]
    assert _estimate(lib, 1, 0, 5)[0] < 0


def test_exl3_layout_matches_reference_tests(lib):
    known = json.load(open(GOLDEN))
    fn = lib.pk_exl3_layout
    fn.argtypes = [ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int32, ctypes.c_void_p]
    fn.restype = ctypes.c_int32
    for case in known["exl3_layout"]["cases"]:
        out = np.zeros(7, np.uint64)
        assert fn(case["in"], case["out"], case["bits"], out.ctypes.data) == 0
        assert [int(v) for v in out[2:5]] == case["trellis_shape"]
        if "trellis_bytes" in case:
            assert int(out[5]) == case["trellis_bytes"] and int(out[6]) == case["scale_bytes"]
    out = np.zeros(7, np.uint64)
    assert fn(4, 4, 0, out.ctypes.data) < 0


def _tile(lib, fmt, epi, m, n):
    fn = lib.pk_gemm_tile
    fn.argtypes = [ctypes.c_int32] * 4 + [ctypes.POINTER(ctypes.c_int32)] * 2
    fn.restype = ctypes.c_int32
    cols, stages = ctypes.c_int32(0), ctypes.c_int32(0)
    rows = fn(fmt, epi, m, n, ctypes.byref(cols), ctypes.byref(stages))
    return rows, cols.value, stages.value


@pytest.mark.skipif(os.environ.get("PK_GEMM_TILE_ROWS") is not None, reason="tile size forced")
def test_gemm_tile_plan(lib):
    """The launcher's tile choice on a 256-CU part (the host-only fallback
    when no GPU is visible, and MI355X's count): the BASELINE sizes the
    full-size parity tests use reach the 256-row kernels; grids of at most
    one tile per CU take the one-tile-per-workgroup ring (more stages)."""
    FP8, I8, G128A8, F16, G128A16, I8SKIP, Q4K = 0, 1, 3, 4, 5, 6, 7
    EPI_F16, EPI_F8, EPI_F32 = 0, 1, 3
    assert _tile(lib, FP8, EPI_F8, 7500, 4096) == (256, 128, 2)
    # 720 tiles of 256 rows would leave the second round of 512 slots 40 % full
    assert _tile(lib, FP8, EPI_F16, 7500, 3072) == (128, 128, 2)
    assert _tile(lib, FP8, EPI_F16, 45000, 3072) == (256, 128, 2)
    assert _tile(lib, FP8, EPI_F16, 45000, 2048) == (256, 128, 2)
    assert _tile(lib, G128A8, EPI_F8, 45000, 4096) == (256, 128, 2)
    assert _tile(lib, FP8, EPI_F16, 45000, 1024) == (256, 128, 2)
    assert _tile(lib, G128A8, EPI_F16, 45000, 1024) == (256, 128, 2)
    assert _tile(lib, I8, EPI_F8, 7500, 4096) == (256, 128, 2)
    assert _tile(lib, FP8, EPI_F16, 7500, 1024) == (128, 128, 2)
    assert _tile(lib, I8SKIP, EPI_F32, 7500, 1024) == (128, 128, 2)
    assert _tile(lib, F16, EPI_F16, 45000, 1024) == (256, 256, 2)
    assert _tile(lib, Q4K, EPI_F16, 16, 256) == (256, 256, 2)
    # small grids: BASELINE config 1 (750 x 4096) in 128-row ring tiles,
    # the T = 750 INT4-g128 FF2 (750 x 1024) in 32-row ring tiles
    rows, cols, stages = _tile(lib, I8, EPI_F32, 750, 4096)
    assert (rows, cols) == (128, 128) and stages >= 3
    rows, cols, stages = _tile(lib, G128A8, EPI_F16, 750, 1024)
    assert (rows, cols) == (32, 128) and stages >= 3
    # the T = 750 INT4-g128 x INT8 FF1 (750 x 4096): 64-row ring tiles, two per CU
    assert _tile(lib, G128A8, EPI_F16, 750, 4096) == (64, 128, 3)
    rows, cols, stages = _tile(lib, I8, EPI_F32, 750, 4096)
    assert (rows, cols) == (128, 128) and stages > 3
    # INT4-g128 x fp16 at 750 x 4096: 96-row ring tiles, 8 x 32 = one per CU
    rows, cols, stages = _tile(lib, G128A16, EPI_F16, 750, 4096)
    assert (rows, cols) == (96, 128) and stages > 3
    assert _tile(lib, 99, EPI_F16, 16, 256)[0] == -4


def test_gemm_k_split(lib):
    """The K split over a ring workgroup's waves: INT4-g128 formats on 32-row
    ring tiles with k >= 1024 only (the T = 750 FF2 of BASELINE config 3)."""
    I8, G128A8, G128A16 = 1, 3, 5
    EPI_F16, EPI_F8, EPI_F32 = 0, 1, 3
    ks = lib.pk_gemm_k_split
    ks.argtypes = [ctypes.c_int32] * 5
    ks.restype = ctypes.c_int32
    assert ks(G128A8, EPI_F32, 750, 1024, 4096) == 4
    assert ks(G128A16, EPI_F16, 750, 1024, 4096) == 4
    assert ks(G128A8, EPI_F8, 97, 1024, 1024) == 4
    assert ks(G128A8, EPI_F32, 750, 1024, 512) == 1    # K too short
    assert ks(G128A8, EPI_F32, 750, 4096, 1024) == 1   # 128-row ring tiles
    assert ks(G128A8, EPI_F16, 45000, 1024, 4096) == 1  # persistent engine
    assert ks(I8, EPI_F32, 750, 1024, 4096) == 1       # not an INT4-g128 format
    assert ks(G128A8, EPI_F32, 750, 0, 4096) == -1
    assert ks(99, EPI_F32, 750, 1024, 4096) == -4


def test_argument_checks_reject_before_any_launch(lib):
    """Entry points reject bad shapes, null and misaligned pointers with their
    PK_E_* code and a message, before touching a device (fake addresses are
    never dereferenced on these paths)."""
    E_SHAPE, E_ALIGN, E_ARG = -1, -2, -4
    vp = ctypes.c_void_p
    err = lib.pk_last_error
    err.restype = ctypes.c_char_p
    ln = lib.pk_layer_norm_quantize_fp8_dynamic
    ln.argtypes = [vp, vp, vp, vp, vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_float, vp]
    ln.restype = ctypes.c_int32
    ok = dict(i=0x10000, w=0x20000, b=0x30000, o=0x40000, s=0x50000)
    assert ln(0x10004, ok["w"], ok["b"], ok["o"], ok["s"], 4, 4, 1e-5, None) == E_ALIGN
    assert b"aligned" in err()
    assert ln(ok["i"], ok["w"], 0x30002, ok["o"], ok["s"], 4, 4, 1e-5, None) == E_ALIGN
    assert ln(ok["i"], ok["w"], ok["b"], 0x40002, ok["s"], 4, 4, 1e-5, None) == E_ALIGN
    assert ln(ok["i"], ok["w"], ok["b"], ok["o"], ok["s"], 5, 4, 1e-5, None) == E_SHAPE
    assert ln(None, ok["w"], ok["b"], ok["o"], ok["s"], 4, 4, 1e-5, None) == E_ARG
    ln4 = lib.pk_layer_norm_quantize_int4_dynamic
    ln4.argtypes = ln.argtypes
    ln4.restype = ctypes.c_int32
    assert ln4(ok["i"], ok["w"], ok["b"], 0x40001, ok["s"], 4, 4, 1e-5, None) == E_ALIGN
    qr = lib.pk_quantize_rows
    qr.argtypes = [ctypes.c_int32, vp, vp, vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, vp]
    qr.restype = ctypes.c_int32
    assert qr(1, 0x10008, ok["o"], ok["s"], 4, 4, 1024, None) == E_ALIGN
    assert qr(1, ok["i"], ok["o"], ok["s"], 4, 4, 1020, None) == E_SHAPE
    assert qr(3, ok["i"], ok["o"], ok["s"], 4, 4, 1024, None) == E_ARG
    assert qr(1, None, ok["o"], ok["s"], 4, 4, 1024, None) == E_ARG
    # exact 2:4 sparse FF2: producer and contract checks
    sq = lib.pk_quantize_rows_int8_sparse24
    sq.argtypes = [vp] * 8 + [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, vp]
    sq.restype = ctypes.c_int32
    assert sq(ok["i"], ok["o"], ok["b"], ok["s"], ok["w"], 0x60000, None, None, 4, 4, 1000, None) == E_SHAPE
    assert sq(ok["i"], ok["o"], ok["b"], ok["s"], ok["w"], 0x60000, None, None, 4, 4, 8192, None) == E_SHAPE
    assert sq(0x10008, ok["o"], ok["b"], ok["s"], ok["w"], 0x60000, None, None, 4, 4, 4096, None) == E_ALIGN
    assert sq(ok["i"], ok["o"], ok["b"], ok["s"], ok["w"], 0x60000, 0x70002, 0x80000, 4, 4, 4096, None) == E_ALIGN
    assert sq(ok["i"], ok["o"], ok["b"], ok["s"], None, 0x60000, None, None, 4, 4, 4096, None) == E_ARG
    assert sq(ok["i"], ok["o"], ok["b"], ok["s"], ok["w"], 0x60000, 0x70000, None, 4, 4, 4096, None) == E_ARG
    assert b"residual" in err()
    sc = lib.pk_ffn_contract_int8_sparse24
    sc.argtypes = [vp] * 11 + [ctypes.c_int32, vp]
    sc.restype = ctypes.c_int32
    args = [0x10000, 0x20000, 0x30000, 0x40000, 0x50000, None, None, 0x60000, 0x70000, 0x80000, 0x90000]
    assert sc(*args, -1, None) == E_SHAPE
    assert sc(*args[:8], None, *args[9:], 8, None) == E_ARG
    assert b"weight_t" in err()
    assert sc(*args[:5], 0xa0000, None, *args[7:], 8, None) == E_ARG
    assert b"residual" in err()
    assert sc(*args[:5], 0xa0000, 0xb0008, *args[7:], 8, None) == E_ALIGN
    assert sc(0x10004, *args[1:], 8, None) == E_ALIGN


def test_unpack_int4_rejects_bad_shapes(lib):
    fn = lib.pk_unpack_int4
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    fn.restype = ctypes.c_int32
    assert fn(None, None, 0, None) == 0          # nothing to do, no GPU work
    assert fn(None, None, 33, None) < 0          # not a multiple of 32
    assert fn(None, None, 64, None) < 0          # missing pointers


def test_fp6_entry_points_reject_before_any_launch(lib):
    """The FP6 form of INT4 codes: pk_gemm format 9 takes only the 2:4 and fp32
    epilogues and k a multiple of 128; the producer, unpack and expand entry
    points check counts, nulls and alignment before touching a device."""
    E_SHAPE, E_ALIGN, E_ARG = -1, -2, -4
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float
    err = lib.pk_last_error
    err.restype = ctypes.c_char_p
    g = lib.pk_gemm
    g.argtypes = [i32, i32, vp, vp, i32, i32, i32, vp, vp, f32, vp, vp, f32, f32, i32, vp, vp, vp, vp, i32, vp]
    g.restype = i32
    args = lambda epi, k: (9, epi, 0x10000, 0x20000, 16, 16, k, None, None, 1.0, None, None, 1.0, 0.0, 0, None, None,
                           0x30000, 0x40000, 16, None)
    assert g(*args(0, 128)) == E_ARG  # fp16 outputs are not a format 9 epilogue
    assert b"unsupported epilogue" in err()
    assert g(*args(3, 64)) == E_SHAPE  # k must be a multiple of 128
    assert b"multiple of 128" in err()
    u = lib.pk_unpack_int4_fp6
    u.argtypes = [vp, vp, ctypes.c_int64, vp]
    u.restype = i32
    assert u(None, None, 0, None) == 0
    assert u(None, None, 33, None) == E_SHAPE
    assert u(None, None, 64, None) == E_ARG
    assert u(0x10008, 0x20000, 64, None) == E_ALIGN
    ln = lib.pk_layer_norm_quantize_int4_fp6
    ln.argtypes = [vp, vp, vp, vp, vp, i32, i32, f32, vp]
    ln.restype = i32
    assert ln(0x10000, 0x20000, 0x30000, 0x40002, 0x50000, 4, 4, 1e-5, None) == E_ALIGN
    assert ln(0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 5, 4, 1e-5, None) == E_SHAPE
    ex = lib.pk_ffn_expand_int4_sparse_fp6
    ex.argtypes = [vp, vp, vp, vp, vp, i32, f32, i32, vp]
    ex.restype = i32
    assert ex(None, 0x20000, 0x30000, 0x40000, 0x50000, 16, 1.0, 1, None) == E_ARG
    assert ex(0x10000, 0x20000, 0x30000, None, 0x50000, 16, 1.0, 1, None) == E_ARG  # dynamic needs input scales
    assert ex(0x10000, 0x20000, 0x30000, 0x40000, 0x50000, -1, 1.0, 1, None) == E_SHAPE
