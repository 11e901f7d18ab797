"""Activation codecs between pipeline stages (runtime/activation/
builtin_activation_codecs.cpp:112-209, activation_codec_factory.cpp:8-46),
through the C ABI on the CPU.

Pinned by the reference's own known answers (activation_codec_test.cpp:
101-176), by every one of the 65536 binary16 patterns (decoding is exact, so
re-encoding must return the pattern; NaNs come back quieted), and by numpy's
independent IEEE float32 -> float16 conversion (round to nearest even) on
values drawn across the normal, subnormal, overflow and tie ranges.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

import jetsonfabric_amd as jf
from jetsonfabric_amd._capi import check


def _enc(values, codec="f16"):
    return jf.activation_encode(np.asarray(values, dtype=np.float32), codec)


def test_reference_known_answers():
    wire = _enc([0.0, -0.0, 1.0, -2.0, 0.3333, 65504.0])
    assert len(wire) == 12  # half the f32 bytes
    back = jf.activation_decode(wire)
    assert back[0] == 0.0 and not math.copysign(1.0, back[0]) < 0
    assert back[1] == 0.0 and math.copysign(1.0, back[1]) < 0
    assert back[2] == 1.0 and back[3] == -2.0
    assert abs(back[4] - 0.3333) < 0.0003
    assert back[5] == 65504.0
    special = jf.activation_decode(_enc([np.inf, -np.inf, np.nan, 2.0**-14, 2.0**-24, 2.0**-25]))
    assert np.isposinf(special[0]) and np.isneginf(special[1]) and np.isnan(special[2])
    assert special[3] == 2.0**-14 and special[4] == 2.0**-24
    assert special[5] == 0.0  # the halfway underflow rounds to even (zero)


def test_f32_codec_is_lossless():
    v = np.random.default_rng(1).standard_normal(257).astype(np.float32)
    wire = jf.activation_encode(v, "f32")
    assert wire == v.tobytes()
    assert np.array_equal(jf.activation_decode(wire, "f32"), v)


def test_every_half_pattern_round_trips():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = jf.activation_decode(h.tobytes())
    # decoding is exact: numpy's float16 -> float32 agrees bit for bit
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(f[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.isnan(f[nan]).all()
    again = np.frombuffer(_enc(f), dtype=np.uint16)
    assert np.array_equal(again[~nan], h[~nan])
    assert np.array_equal(again[nan], h[nan] | 0x0200)  # NaNs quieted, payload kept


def test_matches_numpy_ieee_rounding():
    rng = np.random.default_rng(2)
    parts = [
        rng.standard_normal(20000).astype(np.float32),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),          # subnormal halves
        (rng.uniform(6e4, 7e4, 5000) * rng.choice([-1, 1], 5000)).astype(np.float32),  # overflow edge
        rng.integers(0, 2**32, 50000, dtype=np.uint64).astype(np.uint32).view(np.float32),  # every exponent
    ]
    # exact ties between neighbouring halves: round to even
    h = rng.integers(0, 0x7BFF, 5000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    parts.append(((lo + hi) / 2).astype(np.float32))
    v = np.concatenate(parts)
    v = v[~np.isnan(v)]
    got = np.frombuffer(_enc(v), dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_codec_errors():
    with pytest.raises(jf.JfhError, match="unsupported activation encoding: missing"):
        _enc([1.0], "missing")
    with pytest.raises(jf.JfhError, match="f16 activation byte length must be divisible by two"):
        jf.activation_decode(b"\x00\x01\x02")
    with pytest.raises(jf.JfhError, match="output size does not match"):
        check(jf.library().jfh_activation_encode(b"f16", None, 0, ctypes.create_string_buffer(4), 4))
