"""The C++ .pkl4 reader (pk_artifact_*, host only): a valid artifact's
tensor table, bytes and vocabulary, and every rejection rule of the
reference's validation (artifact.rs:98-157, :514-650)."""
import os
import struct
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "l4-parakeet-rs_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import pkl4_writer as w  # noqa: E402


@pytest.fixture(scope="module")
def pk():
    import parakeet_linear

    return parakeet_linear


def tensors(seed=3):
    rng = np.random.default_rng(seed)
    return [
        ("encoder.layers.0.feed_forward1.linear1.weight", "linear", rng.standard_normal((300, 200)) * 0.02),
        ("encoder.layers.0.feed_forward1.linear1.bias", "bias", rng.standard_normal(300)),
        ("frontend.window", "fp32", rng.standard_normal(17)),
        ("decoder.embedding.weight", "fp16", rng.standard_normal((5, 7))),
    ]


def test_valid_artifact(pk, tmp_path):
    ts = tensors()
    vocab = [f"tok{i}" for i in range(1023)] + ["▁the"]
    path = w.write(tmp_path / "a.pkl4", ts, vocabulary=vocab)
    a = pk.Artifact(str(path))
    info = a.info()
    assert info["profile"] == 0 and info["blank_token_id"] == 1024
    assert info["tensor_count"] == 4 and info["vocabulary_size"] == 1024
    assert info["data_start"] % 4096 == 0 and info["file_bytes"] == info["data_start"] + info["payload_bytes"]
    got = a.tensors()
    assert [t["name"] for t in got] == [t[0] for t in ts]
    assert got[0]["storage"] == "sm89_fp16_linear"
    assert got[0]["logical_shape"] == [300, 200] and got[0]["physical_shape"] == [384, 256]
    assert got[1]["physical_shape"] == [384] and got[1]["bytes"] == 384 * 4
    assert all(t["offset"] % 256 == 0 for t in got)
    # stored bytes: fp16 zero-padded linear (artifact.rs:430-462), fp32 padded bias, plain tensors
    lin = a.read(0).view(np.float16).reshape(384, 256)
    assert np.array_equal(lin[:300, :200], ts[0][2].astype(np.float16))
    assert not lin[300:].any() and not lin[:, 200:].any()
    assert np.array_equal(a.read(1).view(np.float32)[:300], ts[1][2].astype(np.float32))
    assert np.array_equal(a.read(2).view(np.float32), ts[2][2].astype(np.float32))
    assert np.array_equal(a.read(3).view(np.float16).reshape(5, 7), ts[3][2].astype(np.float16))
    assert a.find("frontend.window") == 2
    assert a.vocabulary(1023) == "▁the" and a.vocabulary(1024) is None
    with pytest.raises(pk.PkError, match="missing tensor"):
        a.find("nope")
    a.close()


def _expect(pk, tmp_path, message, **kw):
    path = tmp_path / "bad.pkl4"
    with open(path, "wb") as f:
        f.write(w.build(tensors(), **kw))
    with pytest.raises(pk.PkError, match=message):
        pk.Artifact(str(path))


def _set(key, value):
    return lambda h: h.__setitem__(key, value)


def _tensor(i, key, value):
    return lambda h: h["tensors"][i].__setitem__(key, value)


@pytest.mark.parametrize("kw,message", [
    # artifact.rs:113-140 prefix
    (dict(prefix=lambda v, f, n: (3, f, n)), "expected schema version 2, got 3"),
    (dict(prefix=lambda v, f, n: (v, 1, n)), "unsupported prefix flags"),
    (dict(prefix=lambda v, f, n: (v, f, 0)), "header length 0 is outside"),
    (dict(prefix=lambda v, f, n: (v, f, 100_000_000)), "beyond file length"),
    (dict(prefix=lambda v, f, n: (v, f, n + 9000)), "trailing bytes"),
    # artifact.rs:514-546 header
    (dict(mutate=_set("schema_version", 1)), "header schema is 1"),
    (dict(mutate=_set("target", "gfx950")), "expected sm_89"),
    (dict(mutate=_set("source_revision", "0" * 40)), "profile does not match"),
    (dict(mutate=_set("tensor_alignment", 128)), "tensor alignment is 128"),
    (dict(mutate=_set("payload_bytes", 12)), "payload bytes, file contains"),
    # artifact.rs:594-612 vocabulary
    (dict(vocabulary=["a"] * 1023), "requires 1024 vocabulary entries"),
    (dict(vocabulary=["a"] * 1023 + ["b\tc"]), "control separators"),
    (dict(vocabulary=["a"] * 1023 + [""]), "control separators"),
    # artifact.rs:548-592 tensor table
    (dict(mutate=_tensor(1, "name", "encoder.layers.0.feed_forward1.linear1.weight")), "duplicate tensor name"),
    (dict(mutate=_tensor(2, "offset", 1)), "invalid aligned offset"),
    (dict(mutate=_tensor(3, "bytes", 68)), "header declares 68"),
    (dict(mutate=_tensor(3, "storage", "bf16")), "unknown storage"),
    # artifact.rs:614-650 layouts
    (dict(mutate=_tensor(0, "physical_shape", [300, 256])), "invalid sm_89 FP16 linear shapes"),
    (dict(mutate=_tensor(1, "physical_shape", [300])), "invalid sm_89 FP32 bias shapes"),
    (dict(mutate=_tensor(3, "physical_shape", [7, 5])), "plain storage cannot change"),
])
def test_rejections(pk, tmp_path, kw, message):
    _expect(pk, tmp_path, message, **kw)


def test_rejects_bad_magic_and_short_files(pk, tmp_path):
    data = bytearray(w.build(tensors()))
    data[0:8] = b"PKL4AOX\0"
    (tmp_path / "m.pkl4").write_bytes(bytes(data))
    with pytest.raises(pk.PkError, match="bad magic"):
        pk.Artifact(str(tmp_path / "m.pkl4"))
    (tmp_path / "s.pkl4").write_bytes(b"PKL4")
    with pytest.raises(pk.PkError, match="prefix requires 24"):
        pk.Artifact(str(tmp_path / "s.pkl4"))
    with pytest.raises(pk.PkError, match="failed to open"):
        pk.Artifact(str(tmp_path / "absent.pkl4"))


def test_rejects_payload_past_the_last_tensor(pk, tmp_path):
    # payload_bytes in the header = file payload, but the tensors end earlier
    def grow(h):
        h["payload_bytes"] += 256
    _expect(pk, tmp_path, "payload bytes, file contains", mutate=grow)
    path = tmp_path / "t.pkl4"
    path.write_bytes(w.build(tensors(), mutate=grow, trailing=b"\0" * 256))
    with pytest.raises(pk.PkError, match="last tensor ends at"):
        pk.Artifact(str(path))
