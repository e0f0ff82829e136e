"""Checkpoint ingestion, host side (no GPU): safetensors headers against the ``safetensors``
library as an independent reader, the reference manifest format, the one-read /
two-read rule for (packed, scale) pairs (loader.py:229-266) and the byte counters, and
the fixture encoder (tools/make_synthetic_k3.py:87-110, restated in oracle/mxfp4.py)."""
from __future__ import annotations

import gzip
import json
import struct

import numpy as np
import pytest

from oracle import mxfp4 as om

ck = pytest.importorskip("k3hip.checkpoint")
st = pytest.importorskip("safetensors")


def _some_tensors(rng):
    return {"a.weight": (om.bf16_bits(rng.standard_normal((3, 5)).astype(np.float32)), "BF16"),
            "b.bias": (rng.standard_normal(7).astype(np.float32), "F32"),
            "c.weight_packed": (rng.integers(0, 256, (4, 16), dtype=np.uint8), "U8"),
            "c.weight_scale": (rng.integers(118, 131, (4, 1), dtype=np.uint8), "U8"),
            "d.ids": (np.arange(6, dtype=np.int64).reshape(2, 3), "I64")}


def test_header_and_offsets_match_safetensors_library(tmp_path):
    from safetensors import safe_open
    rng = np.random.default_rng(0)
    tensors = _some_tensors(rng)
    path = tmp_path / "model-00001-of-00001.safetensors"
    ck.write_safetensors(path, tensors)
    recs = ck.scan_checkpoint(tmp_path)
    assert set(recs) == set(tensors)
    raw = path.read_bytes()
    torch = pytest.importorskip("torch")
    with safe_open(str(path), framework="pt") as f:
        for name, (arr, dt) in tensors.items():
            r = recs[name]
            lib = f.get_tensor(name)
            assert list(lib.shape) == r["shape"] == list(arr.shape) and r["dtype"] == dt
            got = raw[r["offset"]:r["offset"] + r["nbytes"]]
            # the library decodes bf16 to torch.bfloat16; compare bit patterns
            want = (lib.view(torch.int16) if dt == "BF16" else lib).numpy().tobytes()
            assert got == want == arr.tobytes()
    # written in the given order, so the pair is adjacent
    assert recs["c.weight_packed"]["offset"] + recs["c.weight_packed"]["nbytes"] == recs["c.weight_scale"]["offset"]


def test_header_guard_rejects_oversized_length(tmp_path):
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(struct.pack("<Q", 10 ** 9) + b"{}")
    with pytest.raises(ValueError, match="header size"):
        ck.read_header(bad)
    short = tmp_path / "short.safetensors"
    short.write_bytes(b"\x01\x02")
    with pytest.raises(ValueError):
        ck.read_header(short)


def test_reference_manifest_resolves_tensors(tmp_path):
    rng = np.random.default_rng(1)
    tensors = _some_tensors(rng)
    ck.write_safetensors(tmp_path / "model-00001-of-00001.safetensors", tensors)
    recs = ck.scan_checkpoint(tmp_path)
    man = tmp_path / "manifest.jsonl.gz"
    with gzip.open(man, "wt") as fh:          # the record layout of k3_manifest.py:104-139
        fh.write(json.dumps({"__meta__": True, "checkpoint": str(tmp_path), "num_experts": 0}) + "\n")
        for r in recs.values():
            fh.write(json.dumps({**r, "component": "text", "layer": None, "role": None}) + "\n")
    src = ck.TensorSource(manifest=man)
    for name, (arr, _) in tensors.items():
        assert np.array_equal(src.host(name), arr)
    assert src.bytes_read == sum(a.nbytes for a, _ in tensors.values())
    with pytest.raises(KeyError):
        src.host("missing.weight")


def test_expert_pair_one_read_when_adjacent_two_otherwise(tmp_path):
    import _synth_ckpt
    ref = _synth_ckpt.make_k3_checkpoint(tmp_path, 5, layer=3, H=128, L=64, I=64, E=4, Is=128, gap_expert=1)
    src = ck.TensorSource(ckpt=tmp_path)
    for e in range(4):
        for j, w in enumerate(("w1", "w3", "w2")):
            r0, b0 = src.reads, src.bytes_read
            p, s = src.expert_host(3, e, w)
            want_p, want_s = ref["experts"][e][j]
            assert np.array_equal(p, want_p) and np.array_equal(s, want_s)
            assert src.reads - r0 == (2 if (e, w) == (1, "w3") else 1)
            assert src.bytes_read - b0 == want_p.nbytes + want_s.nbytes
    assert src.experts_loaded == 12 and src.expert_bytes == src.bytes_read
    with pytest.raises(KeyError):
        src.expert_host(3, 4, "w1")


def test_encoder_is_value_preserving_on_the_grid():
    """Re-encoding decoded MXFP4 reproduces every value: a group whose largest magnitude
    code is 4 or 6 keeps its scale byte and codes; any other group moves to a smaller scale
    with the same values.  A dropped sign, a wrong nibble order or a wrong exponent rule
    changes values."""
    rng = np.random.default_rng(7)
    p, s = om.random_mxfp4(rng, 32, 256)
    w = om.decode_mxfp4(p, s)
    p2, s2 = om.encode_mxfp4(w)
    assert np.array_equal(om.decode_mxfp4(p2, s2), w)
    codes = om.unpack_codes(p).reshape(32, 8, 32) & 7
    top = codes.max(axis=-1) >= 6
    assert np.array_equal(s2[top], s[top])
    assert np.all(s2[~top] <= s[~top])


def test_encoder_known_answers_ties_and_signs():
    """Midpoints between E2M1 magnitudes go to the lower code (numpy argmin's first
    index, make_synthetic_k3.py:104); -0.0 keeps its sign bit (code 8); the group maximum
    lands in [4, 8) times the scale."""
    g = np.zeros((1, 32), np.float32)
    mids = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0]
    g[0, :8] = mids
    g[0, 8:16] = [-m for m in mids]
    g[0, 16] = -0.0
    g[0, 17] = 6.0           # amax 7 -> floor(log2 7) = 2 -> scale byte 127
    p, s = om.encode_mxfp4(g)
    assert s[0, 0] == 127
    codes = om.unpack_codes(p)[0]
    assert list(codes[:8]) == [0, 1, 2, 3, 4, 5, 6, 7]
    assert list(codes[8:16]) == [8, 9, 10, 11, 12, 13, 14, 15]
    assert codes[16] == 8 and codes[17] == 7
    # scale follows the maximum: 48 = 6 * 2^3 -> byte 130, and 0.1 -> 2^(floor(log2 .1)-2)
    p, s = om.encode_mxfp4(np.full((1, 32), 48.0, np.float32))
    assert s[0, 0] == 130 and np.all(om.unpack_codes(p) == 7)
    p, s = om.encode_mxfp4(np.full((1, 32), 0.1, np.float32))
    assert s[0, 0] == 127 + int(np.floor(np.log2(0.1))) - 2
