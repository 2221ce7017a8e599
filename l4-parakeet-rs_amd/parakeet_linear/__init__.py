"""Host-side mirror of the l4-parakeet-rs quantized-linear launch surface.

The reference's Rust host builds each launch with cudarc
(`launch_fp8_linear`, `launch_int8_linear`, `launch_ffn_expand_fp8`, ...;
src/cuda/quant_benchmark.rs:644-745, src/cuda/encoder.rs:1128-1836).  This
module exposes the same operations over the C ABI of libpk_linear.so
(include/pk_linear.h) for torch-allocated device tensors: torch provides the
device memory and the current HIP stream, every computation runs in the HIP
kernels.  There is no fallback: if the library is missing the import fails.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("PK_LINEAR_LIB") or os.path.join(os.path.dirname(HERE), "build", "libpk_linear.so")

P = ctypes.c_void_p
I = ctypes.c_int32
F = ctypes.c_float
S = ctypes.c_size_t

U64 = ctypes.c_uint64


class TensorInfo(ctypes.Structure):
    """pk_tensor_info."""
    _fields_ = [("name", ctypes.c_char_p), ("storage", I), ("rank", I),
                ("logical_shape", U64 * 4), ("physical_shape", U64 * 4),
                ("offset", U64), ("bytes", U64)]


class ArtifactSummary(ctypes.Structure):
    """pk_artifact_summary."""
    _fields_ = [("profile", I), ("blank_token_id", I), ("tensor_count", I),
                ("vocabulary_size", I), ("data_start", U64), ("payload_bytes", U64),
                ("file_bytes", U64)]


# name -> argument types (the trailing stream argument included)
SIGNATURES = {
    "pk_artifact_open": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
    "pk_artifact_close": (None, [P]),
    "pk_artifact_info": (I, [P, ctypes.POINTER(ArtifactSummary)]),
    "pk_artifact_tensor": (I, [P, I, ctypes.POINTER(TensorInfo)]),
    "pk_artifact_find": (I, [P, ctypes.c_char_p]),
    "pk_artifact_vocabulary": (ctypes.c_char_p, [P, I]),
    "pk_artifact_read": (I, [P, I, P, U64]),
    "pk_artifact_derive_linear": (I, [P, I, I, P, U64, P, P, P, P, P]),
    "pk_last_error": (ctypes.c_char_p, []),
    "pk_abi_version": (I, []),
    "pk_estimate_linear": (I, [I, S, S, I, P]),
    "pk_exl3_layout": (I, [S, S, I, P]),
    "pk_pack_fp8_rows": (I, [P, I, I, P, P, P]),
    "pk_pack_int8_rows": (I, [P, I, I, P, P, P]),
    "pk_pack_int4_rows": (I, [P, I, I, P, P, P]),
    "pk_pack_int4_g128": (I, [P, I, I, P, P, P, P]),
    "pk_expand_int4_g128_e4m3": (I, [P, P, P, I, I, P, P, P]),
    "pk_q4_k_dequantize": (I, [P, P, I, I, P]),
    "pk_quantize_fp8": (I, [P, P, F, I, P]),
    "pk_quantize_int8": (I, [P, P, F, I, P]),
    "pk_quantize_fp8_fixed": (I, [P, P, I, F, P]),
    "pk_quantize_rows1024": (I, [P, P, P, I, P]),
    "pk_quantize_rows256": (I, [P, P, P, I, P]),
    "pk_quantize_ffn_contract": (I, [P, P, P, P]),
    "pk_quantize_rows": (I, [I, P, P, P, I, I, I, P]),
    "pk_layer_norm_quantize_fp8_dynamic": (I, [P, P, P, P, P, I, I, F, P]),
    "pk_layer_norm_quantize_int4_dynamic": (I, [P, P, P, P, P, I, I, F, P]),
    "pk_layer_norm_pair": (I, [P, P, P, P, P, P, P, I, I, F, F, P]),
    "pk_layer_norm_quantize_int4_codes": (I, [P, P, P, P, P, I, I, F, P]),
    "pk_unpack_int4": (I, [P, P, ctypes.c_int64, P]),
    "pk_layer_norm_quantize_int4_fp6": (I, [P, P, P, P, P, I, I, F, P]),
    "pk_unpack_int4_fp6": (I, [P, P, ctypes.c_int64, P]),
    "pk_linear_fp16_epilogue": (I, [P, P, P, P, P, I, I, I, F, F, I, P]),
    "pk_linear_fp16_qkv": (I, [P, P, P, P, P, I, I, I, P]),
    "pk_linear_fp8_epilogue": (I, [P, P, P, P, P, I, I, I, F, I, P]),
    "pk_linear_int8_epilogue": (I, [P, P, P, P, P, I, I, I, F, I, P]),
    "pk_linear_int8_accumulate": (I, [P, P, P, I, I, I, P]),
    "pk_linear_int8_dyn": (I, [P, P, P, P, P, P, I, I, I, I, P]),
    "pk_linear_fp8_dyn": (I, [P, P, P, P, P, P, I, I, I, I, P]),
    "pk_linear_int4_accumulate": (I, [P, P, P, I, I, I, P]),
    "pk_linear_int4g128": (I, [P, P, P, P, P, P, I, I, I, I, P]),
    "pk_linear_int4g128_a8": (I, [P, P, P, P, P, P, P, I, I, I, I, P]),
    "pk_q4_k_linear_epilogue": (I, [P, P, P, P, I, I, I, I, P]),
    "pk_ffn_expand_fp8": (I, [P, P, P, P, P, I, F, I, P]),
    "pk_ffn_expand_fp8_packed": (I, [P, P, P, P, P, I, F, I, P]),
    "pk_ffn_expand_int4_sparse": (I, [P, P, P, P, P, I, F, I, P]),
    "pk_ffn_expand_int4_sparse_codes": (I, [P, P, P, P, P, I, F, I, P]),
    "pk_ffn_expand_int4_sparse_fp6": (I, [P, P, P, P, P, I, F, I, P]),
    "pk_ffn_contract_fp8": (I, [P, P, P, P, I, P]),
    "pk_ffn_contract_fp8_sparse": (I, [P, P, P, P, I, I, P]),
    "pk_conv_residual_fp8": (I, [P, P, P, P, P, I, P]),
    "pk_attention_output_fp8": (I, [P, P, P, P, I, P]),
    "pk_conv_glu_fp8": (I, [P, P, P, P, P, I, I, P]),
    "pk_subsample_projection_fp8": (I, [P, P, P, P, P, P, I, P]),
    "pk_subsample_pointwise_fp8": (I, [P, P, P, P, P, P, I, P]),
    "pk_ffn_contract_int8_rowskip": (I, [P, P, P, P, P, I, P, P]),
    "pk_quantize_rows_int8_sparse24": (I, [P, P, P, P, P, P, P, P, I, I, I, P]),
    "pk_transpose_int8": (I, [P, P, I, I, P]),
    "pk_ffn_contract_int8_sparse24": (I, [P, P, P, P, P, P, P, P, P, P, P, I, P]),
    "pk_gemm_k_split": (I, [I, I, I, I, I]),
    "pk_gemm_tile": (I, [I, I, I, I, ctypes.POINTER(I), ctypes.POINTER(I)]),
    "pk_gemm": (I, [I, I, P, P, I, I, I, P, P, F, P, P, F, F, I, P, P, P, P, I, P]),
    "pk_joint_gemv": (I, [P, I, P, P, P, P, P, P, I, I, I, I, I, I, P]),
    "pk_joint_scan": (I, [P, I, P, P, P, P, I, I, I, I, I, I, I, P, P, P]),
    "pk_joint_scan_noalloc": (I, [P, I, P, P, P, P, I, I, I, I, I, I, I, P, P]),
    "pk_tdt_decode_workspace_bytes": (I, [I]),
    "pk_tdt_decode": (I, [P, I, I, P, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I, I, P, I, P, P,
                          ctypes.c_uint64, P]),
    "pk_tdt_decode_long": (I, [P, I, I, P, P, P, P, P, P, P, P, P, P, P, I, P, P, I, I, I, I, P, I, P, P,
                               ctypes.c_uint64, P]),
    "pk_local_relpos_attention": (I, [P, P, P, P, P, P, P, I, I, I, I, I, P]),
    "pk_quantize_fp8_fixed_transpose": (I, [P, P, I, F, P]),
    "pk_pack_position_heads": (I, [P, P, P]),
    "pk_pack_score_vectors": (I, [P, P, P, I, P]),
    "pk_pack_key_int4": (I, [P, P, P, I, P]),
    "pk_quantize_value_int4": (I, [P, P, I, F, P]),
    "pk_quantize_value_int4_register": (I, [P, P, I, F, I, P]),
    "pk_local_relpos_attention_tc_scores": (I, [P, P, P, P, P, P, P, P, I, I, I, I, I, I, P]),
    "pk_local_relpos_attention_packed": (I, [P, P, P, P, P, P, P, P, I, I, I, I, I, I, P, P, P, P, P]),
}


class PkError(RuntimeError):
    pass


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `make -C l4-parakeet-rs_amd` "
            "(or __graft_entry__.build()) first")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    return lib.pk_last_error().decode()


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream=None):
    if stream is not None:
        return stream if isinstance(stream, int) else stream.cuda_stream
    import torch

    return torch.cuda.current_stream().cuda_stream


def call(name: str, *args, stream=None) -> None:
    """Call `name` with tensors converted to device pointers; raise on error."""
    fn = getattr(lib, name)
    conv = []
    for a, t in zip(args, fn.argtypes):
        conv.append(_ptr(a) if t is P else a)
    status = fn(*conv, _stream(stream))
    if status < 0:
        raise PkError(f"{name}: status {status}: {last_error()}")


# ---- reference-named helpers (argument order as in the reference) ----------

def launch_fp8_linear(input, weights, weight_scales, bias, output, m, n, k, input_scale,
                      activation=0, stream=None):
    """quant_benchmark.rs:644-674."""
    call("pk_linear_fp8_epilogue", input, weights, weight_scales, bias, output, m, n, k,
         input_scale, activation, stream=stream)


def launch_int8_linear(input, weights, weight_scales, bias, output, m, n, k, input_scale,
                       activation=0, stream=None):
    """quant_benchmark.rs:677-707."""
    call("pk_linear_int8_epilogue", input, weights, weight_scales, bias, output, m, n, k,
         input_scale, activation, stream=stream)


def launch_linear(input, weights, bias, residual, output, m, n, k, output_scale=1.0,
                  residual_scale=0.0, activation=0, stream=None):
    """cuda.rs:698-740 (launch_linear_view) and the cuBLAS fallback."""
    call("pk_linear_fp16_epilogue", input, weights, bias, residual, output, m, n, k,
         output_scale, residual_scale, activation, stream=stream)


def launch_fp8_quantize(input, output, inverse_scale, stream=None):
    """quant_benchmark.rs:710-727."""
    call("pk_quantize_fp8", input, output, inverse_scale, input.numel(), stream=stream)


def launch_int8_quantize(input, output, inverse_scale, stream=None):
    """quant_benchmark.rs:729-745."""
    call("pk_quantize_int8", input, output, inverse_scale, input.numel(), stream=stream)


def gemm(fmt, epi, a, b, m, n, k, out, *, w_scales=None, row_scales=None, in_scale=1.0,
         bias=None, residual=None, out_scale=1.0, res_scale=0.0, act=0, g_scales=None,
         g_zeros=None, out_meta=None, ldo=None, stream=None):
    call("pk_gemm", fmt, epi, a, b, m, n, k, w_scales, row_scales, in_scale, bias, residual,
         out_scale, res_scale, act, g_scales, g_zeros, out, out_meta, n if ldo is None else ldo,
         stream=stream)


def gemm_tile(fmt, epi, m, n, stages=False):
    """(tile rows, tile cols[, LDS stages]) pk_gemm launches for an m x n output."""
    cols, st = I(0), I(0)
    rows = lib.pk_gemm_tile(fmt, epi, m, n, ctypes.byref(cols), ctypes.byref(st))
    if rows < 0:
        raise PkError(f"pk_gemm_tile: status {rows}: {last_error()}")
    return (rows, cols.value, st.value) if stages else (rows, cols.value)


def gemm_k_split(fmt, epi, m, n, k):
    """K split (1 or 4) of pk_gemm's launch for an m x n x k output."""
    r = lib.pk_gemm_k_split(fmt, epi, m, n, k)
    if r < 0:
        raise PkError(f"pk_gemm_k_split: status {r}: {last_error()}")
    return r


FMT_FP8, FMT_I8, FMT_S4, FMT_G128A8, FMT_F16, FMT_G128A16, FMT_I8_SKIP, FMT_Q4K, FMT_G128F8, FMT_S4F6 = range(10)
EPI_F16, EPI_F8, EPI_F8_24, EPI_F32, EPI_I32 = range(5)


# ---- .pkl4 artifact (host) ------------------------------------------------------

STORAGE = {0: "fp16", 1: "fp32", 2: "sm89_fp16_linear", 3: "sm89_fp32_bias"}
DERIVE_FP16, DERIVE_FP8_ROWS, DERIVE_INT8_ROWS, DERIVE_INT4_ROWS, DERIVE_INT4_G128 = range(5)


class Artifact:
    """An opened, validated .pkl4 artifact (artifact.rs AotArtifactIndex)."""

    def __init__(self, path: str):
        handle = P()
        status = lib.pk_artifact_open(os.fsencode(path), ctypes.byref(handle))
        if status < 0:
            raise PkError(f"pk_artifact_open: status {status}: {last_error()}")
        self.handle = handle.value

    def close(self):
        if getattr(self, "handle", None):
            lib.pk_artifact_close(self.handle)
            self.handle = None

    __del__ = close

    def _check(self, name, status):
        if status < 0:
            raise PkError(f"{name}: status {status}: {last_error()}")
        return status

    def info(self) -> dict:
        out = ArtifactSummary()
        self._check("pk_artifact_info", lib.pk_artifact_info(self.handle, ctypes.byref(out)))
        return {f: getattr(out, f) for f, _ in ArtifactSummary._fields_}

    def tensor(self, index: int) -> dict:
        out = TensorInfo()
        self._check("pk_artifact_tensor", lib.pk_artifact_tensor(self.handle, index, ctypes.byref(out)))
        return {"name": out.name.decode(), "storage": STORAGE[out.storage],
                "logical_shape": list(out.logical_shape[:out.rank]),
                "physical_shape": list(out.physical_shape[:out.rank]),
                "offset": out.offset, "bytes": out.bytes}

    def tensors(self) -> list:
        return [self.tensor(i) for i in range(self.info()["tensor_count"])]

    def find(self, name: str) -> int:
        return self._check("pk_artifact_find", lib.pk_artifact_find(self.handle, name.encode()))

    def vocabulary(self, index: int):
        piece = lib.pk_artifact_vocabulary(self.handle, index)
        return None if piece is None else piece.decode()

    def read(self, index: int):
        import numpy as np

        out = np.empty(self.tensor(index)["bytes"], np.uint8)
        self._check("pk_artifact_read", lib.pk_artifact_read(self.handle, index, out.ctypes.data, out.nbytes))
        return out

    def derive_linear(self, index, fmt, host_staging, device_fp16, packed=None, scales=None, zeros=None,
                      stream=None):
        """Upload tensor `index` (fp16 linear) through `host_staging` (a numpy
        uint8 buffer) into `device_fp16` and pack it on the GPU into `fmt`."""
        fn = lib.pk_artifact_derive_linear
        status = fn(self.handle, index, fmt, host_staging.ctypes.data, host_staging.nbytes,
                    _ptr(device_fp16), _ptr(packed), _ptr(scales), _ptr(zeros), _stream(stream))
        self._check("pk_artifact_derive_linear", status)


# ---- long-form local attention (encoder.rs:1839-1968 launch_attention_arena) ----

ATTENTION_LEFT = ATTENTION_RIGHT = 128
POSITION_ROWS_PADDED = 272


# encoder.rs:619: the fp16 short-form attention below this many padded rows.
SHORT_ATTENTION_ROWS = 512


def cache_position_projection(position_input, position_weight, row_major, output, stream=None):
    """Mirror of one layer of encoder.rs:442-480 (cache_position_projections):
    the fp16 linear of the [272 x 1024] relative-position input with the
    layer's position weight into `row_major`, then pk_pack_position_heads into
    `output` [8 x 272 x 128]."""
    launch_linear(position_input, position_weight, None, None, row_major, POSITION_ROWS_PADDED, 1024, 1024,
                  stream=stream)
    call("pk_pack_position_heads", row_major, output, stream=stream)


def launch_attention_arena(query, key, value_fp8, position, bias_u, bias_v, output, rows, padded_rows,
                           valid_rows, value_stride, packed=None, value=None, stream=None):
    """Mirror of encoder.rs:1839-1968.  With `packed` (padded_rows >= 1040 in
    the reference) it is a dict of caller-owned buffers {key: u8 [padded_rows
    * 512], key_scales: f32 [padded_rows * 8], position: u8 [8 * 272 * 128],
    position_scales: f32 [8 * 272]} that receives the INT4 keys and INT8
    position vectors before pk_local_relpos_attention_packed runs (output e4m3
    bytes); below SHORT_ATTENTION_ROWS padded rows (encoder.rs:619) the fp16
    short-form kernel pk_local_relpos_attention runs on `value` (fp16 [padded_rows
    x 1024]); otherwise pk_local_relpos_attention_tc_scores (output fp16)."""
    if packed is None and padded_rows < SHORT_ATTENTION_ROWS:
        call("pk_local_relpos_attention", query, key, value, position, bias_u, bias_v, output, rows, padded_rows,
             valid_rows, ATTENTION_LEFT, ATTENTION_RIGHT, stream=stream)
        return
    if packed is not None:
        call("pk_pack_key_int4", key, packed["key"], packed["key_scales"], padded_rows * 8, stream=stream)
        call("pk_pack_score_vectors", position, packed["position"], packed["position_scales"], 8 * POSITION_ROWS_PADDED,
             stream=stream)
        call("pk_local_relpos_attention_packed", query, key, None, value_fp8, position, bias_u, bias_v, output, rows,
             padded_rows, valid_rows, ATTENTION_LEFT, ATTENTION_RIGHT, value_stride, packed["key"],
             packed["key_scales"], packed["position"], packed["position_scales"], stream=stream)
    else:
        call("pk_local_relpos_attention_tc_scores", query, key, None, value_fp8, position, bias_u, bias_v, output,
             rows, padded_rows, valid_rows, ATTENTION_LEFT, ATTENTION_RIGHT, value_stride, stream=stream)


# decoder.rs:15: utterances of at least this many frames take the long-request
# decoder (INT8 recurrent weights, layer-0 input table).
LONG_DECODE_MIN_FRAMES = 1024


def launch_decode(encoder_projection, frames, lstm, projection, joint, tokens, result, workspace, *,
                  input_table=None, joint_int8=False, joint_scales=None, hidden=640, token_outputs=1025,
                  durations=5, max_symbols=10, stream=None):
    """Mirror of decoder.rs:275-353 (launch_decode) after the encoder
    projection: for frames >= LONG_DECODE_MIN_FRAMES the layer-0 input table
    (embedding x W_ih0^T, fp16 [token_outputs - 1 x 4H], decoder.rs:355-377) is
    derived with the fp16 linear into `input_table` and pk_tdt_decode_long
    runs; otherwise pk_tdt_decode.  lstm = (embedding, w_ih0, w_hh0, b_ih0,
    b_hh0, w_ih1, w_hh1, b_ih1, b_hh1); projection = (w, b); joint = (w, b).
    Returns "long" or "fp16", the form that ran."""
    emb, w_ih0, w_hh0, b_ih0, b_hh0, w_ih1, w_hh1, b_ih1, b_hh1 = lstm
    capacity = tokens.numel()
    wbytes = workspace.numel() * workspace.element_size()
    if frames >= LONG_DECODE_MIN_FRAMES:
        if input_table is None:
            raise ValueError("the long decode needs an input_table buffer of (token_outputs - 1) x 4H halves")
        launch_linear(emb, w_ih0, None, None, input_table, token_outputs - 1, 4 * hidden, hidden, stream=stream)
        call("pk_tdt_decode_long", encoder_projection, frames, hidden, input_table, w_hh0, b_ih0, b_hh0, w_ih1, w_hh1,
             b_ih1, b_hh1, projection[0], projection[1], joint[0], int(joint_int8), joint_scales, joint[1], hidden,
             token_outputs, durations, max_symbols, tokens, capacity, result, workspace, wbytes, stream=stream)
        return "long"
    call("pk_tdt_decode", encoder_projection, frames, hidden, emb, w_ih0, w_hh0, b_ih0, b_hh0, w_ih1, w_hh1, b_ih1,
         b_hh1, projection[0], projection[1], joint[0], int(joint_int8), joint_scales, joint[1], hidden, token_outputs,
         durations, max_symbols, tokens, capacity, result, workspace, wbytes, stream=stream)
    return "fp16"
