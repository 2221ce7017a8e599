"""Test helper: writes .pkl4 artifacts the way the reference's packer does
(artifact.rs:186-330 plan_fp16, :341-400 write_fp16_artifact), so the C++
reader can be exercised without a checkpoint.  Test infrastructure only.

Layout: b"PKL4AOT\\0", u32 schema 2, u32 flags 0, u64 header length (little
endian), the compact JSON header (serde field order), zero padding to the
first 4096-byte boundary, then each tensor at its 256-byte aligned payload
offset.  Linear weights (fp32 source) become fp16 [ceil128(N) x ceil128(K)]
zero padded; their biases fp32 [ceil128(N)]; other tensors plain fp16/fp32.
"""
import json
import struct

import numpy as np

PROFILES = {  # config.rs:7-10, :41-46
    "v2_english": ("nvidia/parakeet-tdt-0.6b-v2", "ae9ad07059c7c739ffaf932226a8fe64ae2620b0", 1024),
    "v3_multilingual": ("nvidia/parakeet-tdt-0.6b-v3", "541d1f99c6b0c3cd0b11a95167540bb8edefd82b", 8192),
}


def ceil128(v):
    return (v + 127) // 128 * 128


def encode(kind, value):
    """(storage, logical, physical, bytes) of one tensor."""
    value = np.asarray(value)
    if kind == "linear":
        n, k = value.shape
        out = np.zeros((ceil128(n), ceil128(k)), np.float16)
        out[:n, :k] = value.astype(np.float16)
        return "sm89_fp16_linear", [n, k], list(out.shape), out.tobytes()
    if kind == "bias":
        (n,) = value.shape
        out = np.zeros(ceil128(n), np.float32)
        out[:n] = value.astype(np.float32)
        return "sm89_fp32_bias", [n], [ceil128(n)], out.tobytes()
    if kind == "fp32":
        return "fp32", list(value.shape), list(value.shape), value.astype(np.float32).tobytes()
    return "fp16", list(value.shape), list(value.shape), value.astype(np.float16).tobytes()


def build(tensors, profile="v2_english", vocabulary=None, mutate=None, prefix=None, trailing=b""):
    """Bytes of an artifact for [(name, kind, array)].  `mutate(header)` may edit
    the header dict before encoding; `prefix(version, flags, header_len)`
    may replace the prefix fields."""
    repo, rev, blank = PROFILES[profile]
    if vocabulary is None:
        vocabulary = [f"tok{i}" for i in range(blank)]
    records, blobs, cursor = [], [], 0
    for name, kind, value in tensors:
        storage, logical, physical, blob = encode(kind, value)
        cursor = (cursor + 255) // 256 * 256
        records.append({"name": name, "storage": storage, "logical_shape": logical,
                        "physical_shape": physical, "offset": cursor, "bytes": len(blob)})
        blobs.append((cursor, blob))
        cursor += len(blob)
    header = {"schema_version": 2, "target": "sm_89", "profile": profile, "source_repository": repo,
              "source_revision": rev, "source_payload_bytes": cursor, "precision_plan": "fp16",
              "tensor_alignment": 256, "payload_bytes": cursor, "vocabulary": vocabulary,
              "tensors": records}
    if mutate:
        mutate(header)
    text = json.dumps(header, separators=(",", ":"), ensure_ascii=False).encode()
    fields = (2, 0, len(text)) if prefix is None else prefix(2, 0, len(text))
    head = b"PKL4AOT\0" + struct.pack("<IIQ", *fields) + text
    data_start = (len(head) + 4095) // 4096 * 4096
    payload = bytearray(cursor)
    for off, blob in blobs:
        payload[off:off + len(blob)] = blob
    return head + b"\0" * (data_start - len(head)) + bytes(payload) + trailing


def write(path, *args, **kw):
    data = build(*args, **kw)
    with open(path, "wb") as f:
        f.write(data)
    return path
