"""Pins the oracle's block codecs and quantized dot products (CPU only).

The reference stores GGML blocks verbatim (runtime/engines/native/src/
tensor_store.cpp:23-40, 185-196) and leaves the arithmetic to GGML, which is
not present in the checkout. The oracle's dequantization is therefore pinned
here against the published block layouts, written as ENCODERS in this file
(field packing, not decoding), on blocks built from chosen integer codes:

* special blocks with a known answer (unit scales -> y = q; zero blocks;
  maximum codes; one scale/min set per sub-block so that a wrong scale
  index moves a value),
* random codes, with the expected value evaluated in float64 from the codes
  and rounded once to float32 (every K-quant product is exact in float64;
  Q6_K is (d*sc)*q, the rounding order GGML uses),
* the oracle's own quantizer round trip (error within half a step).

The int8 activation scheme (256-value blocks, d = amax/127) is the engine's
own; it is pinned by its round-trip bound and by the integer-exactness of the
quantized dot against a float64 brute force.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import oracle as jo

F16 = np.float16


def f16_bits(x: float) -> int:
    return int(np.array(x, dtype=F16).view(np.uint16))


def f16_val(bits: int) -> float:
    return float(np.array(bits, dtype=np.uint16).view(F16))


# ------------------------------------------------------------------ encoders from the public layouts

def enc_q8_0(d_bits: int, q: np.ndarray) -> bytes:
    """block_q8_0: f16 d, int8 qs[32]."""
    return struct.pack("<H", d_bits) + np.asarray(q, dtype=np.int8).tobytes()


def pack_k4_scales(sc: list[int], mn: list[int]) -> bytes:
    """The 12-byte 6-bit scale/min packing of Q4_K (get_scale_min_k4 inverted)."""
    out = [0] * 12
    for j in range(8):
        if j < 4:
            out[j] |= sc[j] & 63
            out[j + 4] |= mn[j] & 63
        else:
            out[j + 4] |= (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            out[j - 4] |= (sc[j] >> 4) << 6
            out[j] |= (mn[j] >> 4) << 6
    return bytes(out)


def enc_q4_k(d_bits: int, dmin_bits: int, sc: list[int], mn: list[int], q: np.ndarray) -> bytes:
    """block_q4_K: f16 d, f16 dmin, scales[12], qs[128]; sub-block 2p in the low
    nibbles of qs[32p:32p+32], sub-block 2p+1 in the high nibbles."""
    q = np.asarray(q, dtype=np.uint8).reshape(8, 32)
    qs = bytearray(128)
    for p in range(4):
        for l in range(32):
            qs[32 * p + l] = int(q[2 * p, l]) | (int(q[2 * p + 1, l]) << 4)
    return struct.pack("<HH", d_bits, dmin_bits) + pack_k4_scales(sc, mn) + bytes(qs)


def q6_position(i: int) -> tuple[int, int, int, int]:
    """(ql byte, ql shift, qh byte, qh shift) of value i in block_q6_K."""
    half, w = divmod(i, 128)
    quarter, l = divmod(w, 32)
    ql = 64 * half + l + (32 if quarter in (1, 3) else 0)
    return ql, 4 if quarter >= 2 else 0, 32 * half + l, 2 * quarter


def enc_q6_k(d_bits: int, sc: list[int], q: np.ndarray) -> bytes:
    """block_q6_K: ql[128], qh[64], int8 scales[16], f16 d; value = q - 32 with
    q a 6-bit code, scale index i/16."""
    ql = bytearray(128)
    qh = bytearray(64)
    for i in range(256):
        code = int(q[i])
        a, sa, b, sb = q6_position(i)
        ql[a] |= (code & 0xF) << sa
        qh[b] |= (code >> 4) << sb
    return bytes(ql) + bytes(qh) + np.asarray(sc, dtype=np.int8).tobytes() + struct.pack("<H", d_bits)


def q2_position(i: int) -> tuple[int, int]:
    """(qs byte, shift) of value i in block_q2_K: halves of 128, four 2-bit
    planes of 32 values each."""
    half, w = divmod(i, 128)
    plane, l = divmod(w, 32)
    return 32 * half + l, 2 * plane


def enc_q2_k(d_bits: int, dmin_bits: int, sc: list[int], mn: list[int], q: np.ndarray) -> bytes:
    """block_q2_K: scales[16] (scale low nibble, min high nibble), qs[64], f16 d, f16 dmin;
    value i uses scale byte i/16."""
    qs = bytearray(64)
    for i in range(256):
        b, s = q2_position(i)
        qs[b] |= (int(q[i]) & 3) << s
    scales = bytes((sc[j] & 0xF) | ((mn[j] & 0xF) << 4) for j in range(16))
    return scales + bytes(qs) + struct.pack("<HH", d_bits, dmin_bits)


# ------------------------------------------------------------------ expected values (float64, one rounding)

def exp_q8_0(d_bits, q):
    return (f16_val(d_bits) * np.asarray(q, dtype=np.float64)).astype(np.float32)


def exp_q4_k(d_bits, dmin_bits, sc, mn, q):
    q = np.asarray(q, dtype=np.float64).reshape(8, 32)
    d, dm = f16_val(d_bits), f16_val(dmin_bits)
    return np.concatenate([d * sc[j] * q[j] - dm * mn[j] for j in range(8)]).astype(np.float32)


def exp_q6_k(d_bits, sc, q):
    q = np.asarray(q, dtype=np.float64) - 32.0
    d = f16_val(d_bits)
    return np.array([(d * sc[i // 16]) * q[i] for i in range(256)]).astype(np.float32)


def exp_q2_k(d_bits, dmin_bits, sc, mn, q):
    q = np.asarray(q, dtype=np.float64)
    d, dm = f16_val(d_bits), f16_val(dmin_bits)
    return np.array([d * sc[i // 16] * q[i] - dm * mn[i // 16] for i in range(256)]).astype(np.float32)


def deq(type_id: int, data: bytes) -> np.ndarray:
    e, b = jo.block(type_id)
    return jo.dequantize_row(type_id, data, len(data) // b * e)


# ------------------------------------------------------------------ block table

def test_block_table_matches_ggml_layouts():
    # engine.c:292-303 / docs/jfm-v2-format.md:83-90
    assert jo.block(jo.F32) == (1, 4)
    assert jo.block(jo.F16) == (1, 2)
    assert jo.block(jo.Q8_0) == (32, 34)
    assert jo.block(jo.Q2_K) == (256, 84)
    assert jo.block(jo.Q4_K) == (256, 144)
    assert jo.block(jo.Q6_K) == (256, 210)


@pytest.mark.skipif(not jo.ref_loader.available(), reason="reference loader not built (oracle/_ref)")
def test_block_table_matches_reference_loader():
    for t in (jo.F32, jo.F16, jo.Q8_0, jo.Q2_K, jo.Q4_K, jo.Q6_K):
        assert jo.ref_loader.type_layout(t) == jo.block(t)


def test_f16_conversion_is_ieee_binary16():
    for x in [0.0, 1.0, -2.5, 65504.0, 6.1035156e-05, 5.9604645e-08, 0.1, 1e-3]:
        assert jo.f32_to_f16(x) == f16_bits(x)
        assert jo.f16_to_f32(f16_bits(x)) == np.float32(np.float16(x))
    # every finite binary16 code decodes exactly; rounding ties go to even
    codes = np.arange(65536, dtype=np.uint16)
    vals = codes.view(F16).astype(np.float32)
    for c in range(65536):
        if np.isfinite(vals[c]):
            assert jo.f16_to_f32(int(c)) == vals[c], c
    rng = np.random.default_rng(3)
    for x in np.concatenate([rng.standard_normal(500) * 10.0, rng.standard_normal(200) * 1e-5]).astype(np.float32):
        assert jo.f32_to_f16(float(x)) == f16_bits(x), x
    halfway = np.float32(1.0 + 2.0 ** -11)  # between 1.0 and the next binary16 value: ties to even (1.0)
    assert jo.f32_to_f16(float(halfway)) == f16_bits(1.0)


# ------------------------------------------------------------------ special blocks

def test_q8_0_unit_and_zero_blocks():
    q = np.arange(-16, 16)
    assert np.array_equal(deq(jo.Q8_0, enc_q8_0(f16_bits(1.0), q)), q.astype(np.float32))
    assert not deq(jo.Q8_0, enc_q8_0(0, q)).any()
    extremes = np.array([-128, 127] * 16)
    assert np.array_equal(deq(jo.Q8_0, enc_q8_0(f16_bits(0.5), extremes)), extremes * 0.5)


def test_q4_k_scale_and_min_index_mapping():
    # unit scales, zero mins: y == q
    q = np.arange(256) % 16
    ones = [1] * 8
    got = deq(jo.Q4_K, enc_q4_k(f16_bits(1.0), 0, ones, [0] * 8, q))
    assert np.array_equal(got, q.astype(np.float32))
    # distinct 6-bit scales and mins per sub-block (j >= 4 exercise the split high bits)
    sc = [1, 7, 33, 63, 2, 48, 17, 62]
    mn = [0, 5, 63, 31, 61, 3, 40, 9]
    got = deq(jo.Q4_K, enc_q4_k(f16_bits(1.0), f16_bits(1.0), sc, mn, np.full(256, 1)))
    for j in range(8):
        assert np.all(got[32 * j:32 * j + 32] == sc[j] - mn[j]), j
    # maximum codes
    got = deq(jo.Q4_K, enc_q4_k(f16_bits(2.0), f16_bits(0.5), [63] * 8, [63] * 8, np.full(256, 15)))
    assert np.all(got == 2.0 * 63 * 15 - 0.5 * 63)
    assert not deq(jo.Q4_K, bytes(144)).any()


def test_q6_k_value_and_scale_positions():
    # each value gets a distinct code; unit scale: y == code - 32
    q = (np.arange(256) * 7) % 64
    got = deq(jo.Q6_K, enc_q6_k(f16_bits(1.0), [1] * 16, q))
    assert np.array_equal(got, (q - 32).astype(np.float32))
    # one scale per 16 values, signed
    sc = [(-1) ** j * (j + 1) for j in range(16)]
    got = deq(jo.Q6_K, enc_q6_k(f16_bits(1.0), sc, np.full(256, 33)))
    for j in range(16):
        assert np.all(got[16 * j:16 * j + 16] == sc[j]), j
    assert np.all(deq(jo.Q6_K, enc_q6_k(f16_bits(1.0), [127] * 16, np.zeros(256))) == -32 * 127)


def test_q2_k_value_and_scale_positions():
    q = (np.arange(256) // 3) % 4
    got = deq(jo.Q2_K, enc_q2_k(f16_bits(1.0), 0, [1] * 16, [0] * 16, q))
    assert np.array_equal(got, q.astype(np.float32))
    sc = [(j % 15) + 1 for j in range(16)]
    mn = [15 - j for j in range(16)]
    got = deq(jo.Q2_K, enc_q2_k(f16_bits(1.0), f16_bits(1.0), sc, mn, np.full(256, 2)))
    for j in range(16):
        assert np.all(got[16 * j:16 * j + 16] == 2 * sc[j] - mn[j]), j


# ------------------------------------------------------------------ random codes, float64 expected values

def _rand_f16(rng, lo=1e-4, hi=0.05):
    return f16_bits(float(rng.uniform(lo, hi)))


@pytest.mark.parametrize("seed", range(8))
def test_random_blocks_bit_exact(seed):
    rng = np.random.default_rng(seed)
    for _ in range(16):
        d, dm = _rand_f16(rng), _rand_f16(rng)
        q = rng.integers(-128, 128, 32)
        assert np.array_equal(deq(jo.Q8_0, enc_q8_0(d, q)), exp_q8_0(d, q))

        sc, mn, q = list(rng.integers(0, 64, 8)), list(rng.integers(0, 64, 8)), rng.integers(0, 16, 256)
        assert np.array_equal(deq(jo.Q4_K, enc_q4_k(d, dm, sc, mn, q)), exp_q4_k(d, dm, sc, mn, q))

        sc6, q6 = list(rng.integers(-128, 128, 16)), rng.integers(0, 64, 256)
        assert np.array_equal(deq(jo.Q6_K, enc_q6_k(d, sc6, q6)), exp_q6_k(d, sc6, q6))

        sc2, mn2, q2 = list(rng.integers(0, 16, 16)), list(rng.integers(0, 16, 16)), rng.integers(0, 4, 256)
        assert np.array_equal(deq(jo.Q2_K, enc_q2_k(d, dm, sc2, mn2, q2)), exp_q2_k(d, dm, sc2, mn2, q2))


def test_multi_block_rows_decode_block_by_block():
    rng = np.random.default_rng(99)
    blocks, expected = [], []
    for _ in range(5):
        d, dm = _rand_f16(rng), _rand_f16(rng)
        sc, mn, q = list(rng.integers(0, 64, 8)), list(rng.integers(0, 64, 8)), rng.integers(0, 16, 256)
        blocks.append(enc_q4_k(d, dm, sc, mn, q))
        expected.append(exp_q4_k(d, dm, sc, mn, q))
    assert np.array_equal(deq(jo.Q4_K, b"".join(blocks)), np.concatenate(expected))


# ------------------------------------------------------------------ quantizer round trip (synthetic weights)

@pytest.mark.parametrize("type_id,rel", [(jo.Q8_0, 0.01), (jo.Q6_K, 0.04), (jo.Q4_K, 0.15), (jo.Q2_K, 0.6)])
def test_synthesized_weights_round_trip(type_id, rel):
    import jetsonfabric_amd as jf

    cfg = jf.ModelConfig(n_layer=1, n_embd=512, n_ff=512, n_head=4, n_head_kv=2, n_vocab=512, n_ctx=64)
    m = jf.Model.synthesize(cfg, type_linear=type_id, type_embd=type_id, type_output=type_id, seed=5)
    raw = m.tensor_bytes("blk.0.attn_q.weight")
    w = deq(type_id, raw)
    assert w.size == 512 * 512
    # N(0, 0.02) weights: dequantized std within the type's relative error of 0.02
    assert abs(float(np.std(w)) - 0.02) < 0.02 * rel + 1e-3
    assert abs(float(np.mean(w))) < 2e-3


# ------------------------------------------------------------------ activation quantization and dots

def test_activation_quantization_round_trip():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, 1024).astype(np.float32)
    x[256:512] = 0.0
    q, d, s = jo.quantize_act(x)
    assert d[1] == 0.0 and not q[256:512].any()
    for b in range(4):
        blk = x[256 * b:256 * b + 256]
        assert d[b] == np.float32(np.abs(blk).max()) / np.float32(127.0)
        if d[b] > 0:
            err = np.abs(q[256 * b:256 * b + 256].astype(np.float64) * d[b] - blk)
            assert err.max() <= 0.5 * d[b] * (1 + 1e-6)
            assert np.abs(q[256 * b:256 * b + 256]).max() == 127
    assert np.array_equal(s, q.astype(np.int32).reshape(-1, 16).sum(axis=1))


def test_activation_quantization_32_value_blocks():
    """The 32-value rule (GGML's q8_0 / q8_1 block): per block d' = amax/127,
    codes roundf(x / d') from the f32 scale, stored scale d' rounded to f16
    (numpy's IEEE conversion); every code within half a step of x plus the
    scale's f16 rounding, and 16-value code sums."""
    rng = np.random.default_rng(31)
    x = rng.normal(0, 2, 1024).astype(np.float32)
    x[64:96] = 0.0                      # a zero block
    x[96:128] *= np.float32(1e-3)       # a small block: f16 scale well inside the normal range
    x[128:160] = np.float32(-7.0)       # a constant block: every code -127
    q, d, s = jo.quantize_act(x, 32)
    assert d.size == 32
    for b in range(32):
        blk = x[32 * b:32 * b + 32]
        d_raw = np.float32(np.abs(blk).max()) / np.float32(127.0)
        assert d[b] == np.float32(np.float16(d_raw)), f"block {b}"
        codes = q[32 * b:32 * b + 32].astype(np.float64)
        if d_raw == 0:
            assert not codes.any()
            continue
        assert np.abs(codes).max() == 127
        assert np.array_equal(codes, np.clip(np.round(blk.astype(np.float64) / float(d_raw)), -127, 127)) or \
            np.abs(codes - blk / float(d_raw)).max() <= 0.5 + 1e-5
        err = np.abs(codes * float(d[b]) - blk)
        assert err.max() <= 0.5 * float(d_raw) * (1 + 1e-5) + 127 * abs(float(d[b]) - float(d_raw))
    assert np.all(q[128:160] == -127)
    assert np.array_equal(s, q.astype(np.int32).reshape(-1, 16).sum(axis=1))
    # 32-value blocks never quantize more coarsely than the 256-value rule
    q256, d256, _ = jo.quantize_act(x)
    e32 = np.abs(q.astype(np.float64) * np.repeat(d.astype(np.float64), 32) - x)
    e256 = np.abs(q256.astype(np.float64) * np.repeat(d256.astype(np.float64), 256) - x)
    assert e32.mean() < e256.mean()


def test_normalized_activation_quantization():
    """jfo_quantize_act_normed against the definition of the rule: the codes
    are those of x * gain (one scale per 256 values, amax / 127), each block
    scale is then multiplied by the row's 1 / sqrtf(mean(x^2) + eps), so the
    dequantized codes reproduce RMSNorm(x) * gain (qwen2_architecture.cpp:
    373-376) to half a code step."""
    rng = np.random.default_rng(8)
    n, eps = 1024, 1e-6
    x = rng.normal(0, 3, n).astype(np.float32)
    gain = rng.uniform(0.5, 1.5, n).astype(np.float32)
    gain[512:768] = 0.0  # one block of zero gains: zero codes, zero scale
    q, d, s = jo.quantize_act_normed(x, gain, eps)
    rs = np.float32(1.0) / np.sqrt(np.float32(np.sum(x.astype(np.float64) ** 2) / n) + np.float32(eps))
    normed = (x.astype(np.float64) * float(rs)) * gain.astype(np.float64)
    v = x * gain  # float32 products, the quantized values before normalization
    for b in range(n // 256):
        blk = slice(256 * b, 256 * b + 256)
        d_unnormed = np.float32(np.abs(v[blk]).max()) / np.float32(127.0)
        assert d[b] == np.float32(d_unnormed * rs), f"block {b} scale"
        if d[b] == 0:
            assert not q[blk].any()
            continue
        assert np.abs(q[blk]).max() == 127
        err = np.abs(q[blk].astype(np.float64) * float(d[b]) - normed[blk])
        assert err.max() <= 0.5 * float(d[b]) * (1 + 1e-5), f"block {b}: {err.max()} vs step {d[b]}"
    assert d[2] == 0.0
    assert np.array_equal(s, q.astype(np.int32).reshape(-1, 16).sum(axis=1))
    # the unnormalized rule on x * gain gives the same codes
    q2, d2, _ = jo.quantize_act(v)
    assert np.array_equal(q, q2) and np.array_equal(d, (d2 * rs).astype(np.float32))
    # 32-value blocks: the codes of x * gain per 32 values, the scale
    # (amax / 127 * rs) rounded to f16
    q32, d32, s32 = jo.quantize_act_normed(x, gain, eps, 32)
    for b in range(n // 32):
        blk = slice(32 * b, 32 * b + 32)
        d_raw = np.float32(np.abs(v[blk]).max()) / np.float32(127.0)
        assert d32[b] == np.float32(np.float16(np.float32(d_raw * rs))), f"block {b}"
        if d_raw > 0:
            assert np.abs(q32[blk].astype(np.float64) - v[blk] / float(d_raw)).max() <= 0.5 + 1e-5
            err = np.abs(q32[blk].astype(np.float64) * float(d32[b]) - normed[blk])
            assert err.max() <= 0.5 * float(d_raw * rs) * (1 + 1e-5) + 127 * abs(float(d32[b]) - float(d_raw * rs))
        else:
            assert not q32[blk].any()
    assert np.array_equal(s32, q32.astype(np.int32).reshape(-1, 16).sum(axis=1))


@pytest.mark.parametrize("type_id", [jo.Q8_0, jo.Q2_K, jo.Q4_K, jo.Q6_K])
def test_quantized_dot_equals_float64_brute_force(type_id):
    """vec_dot_q8 = sum over blocks of exact integer sums -> equals
    sum_i dequant(w)_i * (q_i * d_blk) evaluated in float64, with the type's
    activation blocks (256 values for the K-quants, 32 for Q8_0: GGML's
    q8_0 x q8_0 rule)."""
    blk = jo.act_block(type_id)
    rng = np.random.default_rng(type_id + blk)
    n = 1024
    _, bb = jo.block(type_id)
    e, _ = jo.block(type_id)
    row = rng.integers(0, 256, n // e * bb, dtype=np.uint8)
    # keep f16 scales finite and small: overwrite the scale fields with chosen values
    row = bytearray(row.tobytes())
    for b in range(n // e):
        o = b * bb
        if type_id == jo.Q8_0:
            row[o:o + 2] = struct.pack("<H", _rand_f16(rng))
        elif type_id == jo.Q4_K:
            row[o:o + 4] = struct.pack("<HH", _rand_f16(rng), _rand_f16(rng))
        elif type_id == jo.Q2_K:
            row[o + 80:o + 84] = struct.pack("<HH", _rand_f16(rng), _rand_f16(rng))
        else:
            row[o + 208:o + 210] = struct.pack("<H", _rand_f16(rng))
    row = bytes(row)
    w = deq(type_id, row).astype(np.float64)
    x = rng.normal(0, 1, n).astype(np.float32)
    q, d, s = jo.quantize_act(x, blk)
    xq = q.astype(np.float64) * np.repeat(d.astype(np.float64), blk)
    expected = float(w @ xq)
    got = jo.vec_dot_q8(type_id, row, q, d, s, blk)
    assert got == pytest.approx(expected, rel=1e-6, abs=1e-6 * float(np.abs(w) @ np.abs(xq)))
    exact = jo.vec_dot_f32(type_id, row, x)
    assert exact == pytest.approx(float(w @ x.astype(np.float64)), rel=1e-9, abs=1e-9)
    # the wrong block size is refused (Q8_0 takes 32-value blocks, the K-quants 256)
    other = 256 if blk == 32 else 32
    q2, d2, s2 = jo.quantize_act(x, other)
    assert jo.vec_dot_q8(type_id, row, q2, d2, s2, other) == 0.0
    if blk == 32:
        # a planted mistake the comparison above must catch: the scales of two blocks exchanged
        bad = d.copy()
        bad[[3, 4]] = bad[[4, 3]]
        assert bad[3] != bad[4]
        wrong = jo.vec_dot_q8(type_id, row, q, bad, s, blk)
        assert abs(wrong - expected) > 1e-6 * float(np.abs(w) @ np.abs(xq))


def test_matmul_modes_agree_with_brute_force():
    import jetsonfabric_amd as jf

    cfg = jf.ModelConfig(n_layer=1, n_embd=512, n_ff=512, n_head=4, n_head_kv=2, n_vocab=512, n_ctx=64)
    m = jf.Model.synthesize(cfg, type_linear=jo.Q4_K, type_embd=jo.Q4_K, type_output=jo.Q6_K, seed=8)
    raw = m.tensor_bytes("blk.0.attn_q.weight")
    w = deq(jo.Q4_K, raw).reshape(512, 512).astype(np.float64)
    x = np.random.default_rng(1).normal(0, 1, (3, 512)).astype(np.float32)
    exact = jo.matmul(jo.Q4_K, raw, 512, 512, x, jo.MODE_EXACT, 2)
    assert np.allclose(exact, x.astype(np.float64) @ w.T, rtol=1e-5, atol=1e-5)
    q8 = jo.matmul(jo.Q4_K, raw, 512, 512, x, jo.MODE_Q8, 2)
    # int8 activations: error bounded by half a step per value
    bound = 0.5 * np.abs(w).sum(axis=1)[None, :] * (np.abs(x).max(axis=1, keepdims=True) / 127.0)
    assert np.all(np.abs(q8 - exact) <= bound + 1e-6)
    assert jo.nrmse(exact, q8) < 1e-2
