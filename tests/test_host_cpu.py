"""Host-side pieces of the driver and loader, on the CPU: top-k sampling
(generate_tinyllama.py:124-143) and safetensors files with BF16-stored
tensors (the header/offset layout of coreml_backend.py:21-54)."""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from chomikgrad.dtypes import BFLOAT16, bf16_to_float32
from chomikgrad.hip_backend import read_safetensors
from chomikgrad.runtime import sample_token


def test_sampling_temperature_zero_is_first_argmax():
    logits = np.array([[0.5, 3.0, -1.0, 3.0]], np.float32)
    assert sample_token(logits, temperature=0, top_k=2, rng=np.random.default_rng(0)) == 1


def test_sampling_top1_is_argmax_for_any_draw():
    logits = np.array([[0.1, 0.3, 2.0, -0.5, 1.9]], np.float32)
    for seed in range(20):
        assert sample_token(logits, temperature=1.7, top_k=1, rng=np.random.default_rng(seed)) == 2


def test_sampling_top2_closed_form_draw():
    """Logits (2, 1, 0, -1) at temperature 1, top_k 2: the kept entries are 0
    and 1 with probabilities e/(e+1) and 1/(e+1) (closed form).  NumPy's
    Generator.choice with p draws one uniform u and returns the first index
    whose cumulative probability exceeds it, so each seed's token follows
    from its u."""
    logits = np.array([[2.0, 1.0, 0.0, -1.0]], np.float32)
    p0 = np.e / (np.e + 1)
    seen = set()
    for seed in range(40):
        u = np.random.default_rng(seed).random()
        expected = 0 if u < p0 else 1
        got = sample_token(logits, temperature=1.0, top_k=2, rng=np.random.default_rng(seed))
        assert got == expected, seed
        seen.add(got)
    assert seen == {0, 1}


def test_sampling_frequencies_follow_tempered_softmax():
    """20000 draws over the top 3 of 6 logits at temperature 0.5: tokens outside
    the top 3 never appear, and the frequencies of the kept ones match
    softmax(logit / 0.5) over those three within 4 standard errors."""
    logits = np.array([[0.2, 1.0, -3.0, 0.7, 0.1, 1.2]], np.float32)
    rng = np.random.default_rng(11)
    draws = np.array([sample_token(logits, temperature=0.5, top_k=3, rng=rng) for _ in range(20000)])
    assert set(np.unique(draws)) <= {1, 3, 5}
    kept = np.array([1.0, 0.7, 1.2]) / 0.5
    p = np.exp(kept - kept.max()) / np.exp(kept - kept.max()).sum()
    freq = np.array([np.mean(draws == i) for i in (1, 3, 5)])
    assert np.all(np.abs(freq - p) < 4 * np.sqrt(p * (1 - p) / draws.size))


def write_safetensors(path, entries):
    """entries: name -> (dtype tag, shape, raw bytes)."""
    header, blobs, offset = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (tag, shape, raw) in entries.items():
        header[name] = {"dtype": tag, "shape": list(shape), "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    blob = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(blob)) + blob + b"".join(blobs))


BF16_BITS = np.array([0x3F80, 0xC020, 0x4049, 0x0001, 0x7F7F, 0xFF80, 0x8000, 0x3E80], np.uint16)
BF16_VALUES = np.array([1.0, -2.5, 3.140625, 9.183549615799121e-41, 3.3895313892515355e38, -np.inf, -0.0, 0.25],
                       np.float32)


def test_bf16_stored_tensor_is_read_bit_exactly(tmp_path):
    """A BF16-stored tensor: kept as bfloat16 bits, widened exactly to float32,
    rounded to float16 on request (subnormal -> 0, above 65504 -> inf)."""
    path = tmp_path / "w.safetensors"
    write_safetensors(path, {"w": ("BF16", (2, 4), BF16_BITS.tobytes()),
                             "f": ("F32", (3,), np.array([1.5, -2.0, 0.1], np.float32).tobytes())})
    raw = read_safetensors(path)
    assert raw["w"].dtype == BFLOAT16 and raw["w"].shape == (2, 4)
    np.testing.assert_array_equal(raw["w"].view(np.uint16).reshape(-1), BF16_BITS)
    np.testing.assert_array_equal(bf16_to_float32(raw["w"]).reshape(-1), BF16_VALUES)
    widened = read_safetensors(path, np.float32)
    assert widened["w"].dtype == np.float32
    np.testing.assert_array_equal(widened["w"].reshape(-1), BF16_VALUES)
    narrowed = read_safetensors(path, np.float16)["w"].reshape(-1)
    np.testing.assert_array_equal(narrowed, BF16_VALUES.astype(np.float16))
    assert narrowed[3] == 0 and np.isinf(narrowed[4])


def test_inconsistent_offsets_are_rejected(tmp_path):
    path = tmp_path / "bad.safetensors"
    write_safetensors(path, {"w": ("BF16", (3,), BF16_BITS[:2].tobytes())})
    with pytest.raises(ValueError):
        read_safetensors(path)
