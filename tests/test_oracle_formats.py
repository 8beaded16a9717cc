"""Pins the oracle's block formats: f16 conversions, dequant, quantize.

Checks are closed forms, known answers and the reference's own invariant
tests (src/quant.rs:513-606), chosen so that a wrong offset, scale, nibble
pairing, bit-plane position or rounding rule fails one of them.
"""
import numpy as np
import pytest

Q4, Q5, Q8, F32, F16 = 2, 6, 8, 0, 1


def test_f16_to_f32_every_value(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rounding_rules(oracle):
    rng = np.random.default_rng(0)
    # Normal range: round to nearest even, same as IEEE (numpy).
    x = (rng.standard_normal(200000) * np.exp2(rng.integers(-14, 15, 200000))).astype(np.float32)
    x = x[(np.abs(x) < 65504) & (np.abs(x) >= 2.0**-14)]
    assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16))
    # Subnormal results truncate to 13 fraction bits below the new binary
    # point, then round half UP (src/quant.rs:160-166), unlike IEEE:
    # 2.5 * 2^-24 -> 3 * 2^-24, where round-to-even gives 2 * 2^-24.
    tie = np.float32(2.5 * 2.0**-24)
    assert oracle.f32_to_f16(np.array([tie]))[0] == 3
    assert np.float16(tie).view(np.uint16) == 2
    assert oracle.f32_to_f16(np.array([np.float32(3.5 * 2.0**-24)]))[0] == 4
    # Below half the smallest subnormal -> signed zero; overflow and NaN -> inf.
    assert oracle.f32_to_f16(np.array([np.float32(-2.0**-26)]))[0] == 0x8000
    assert oracle.f32_to_f16(np.array([np.float32(70000.0), np.float32(np.nan)])).tolist() == [0x7C00, 0x7C00]
    # A mantissa carry bumps the exponent: 2047.9 -> 2048.
    assert oracle.f16_to_f32(oracle.f32_to_f16(np.array([np.float32(2047.9)])))[0] == 2048.0


def test_row_bytes_and_bits_per_weight(oracle):
    for dt, per_block, bits in [(Q4, 18, 4.5), (Q5, 22, 5.5), (Q8, 34, 8.5)]:
        assert oracle.row_bytes(dt, 32) == per_block
        assert oracle.row_bytes(dt, 4096) == 128 * per_block
        assert per_block * 8 / 32 == bits
    assert oracle.row_bytes(F32, 7) == 28


def _block(scale_bits: int, payload: bytes) -> np.ndarray:
    return np.frombuffer(scale_bits.to_bytes(2, "little") + payload, dtype=np.uint8)


@pytest.mark.parametrize("scale", [0x3C00, 0x2E66, 0x0001, 0x8400, 0x5BFF])
def test_dequant_closed_form(oracle, scale):
    d = np.float32(np.uint16(scale).view(np.float16))
    # Q8: every int8 code.
    codes = np.arange(256, dtype=np.uint8)
    for chunk in range(8):
        c = codes[chunk * 32:(chunk + 1) * 32]
        got = oracle.dequant(Q8, _block(scale, c.tobytes()), 1, 32)[0]
        assert np.array_equal(got, d * c.view(np.int8).astype(np.float32))
    # Q4: byte i holds element i (low nibble) and i + 16 (high nibble).
    for base in range(0, 256, 16):
        b = np.arange(base, base + 16, dtype=np.uint8)
        got = oracle.dequant(Q4, _block(scale, b.tobytes()), 1, 32)[0]
        want = np.concatenate([(b & 15).astype(np.float32) - 8, (b >> 4).astype(np.float32) - 8]) * d
        assert np.array_equal(got, want)
    # Q5: a little-endian 32-bit plane of high bits before the nibbles.
    rng = np.random.default_rng(scale)
    for _ in range(16):
        plane = int(rng.integers(0, 2**32))
        nib = rng.integers(0, 256, 16, dtype=np.uint8)
        got = oracle.dequant(Q5, _block(scale, plane.to_bytes(4, "little") + nib.tobytes()), 1, 32)[0]
        lo = np.concatenate([nib & 15, nib >> 4]).astype(np.int32)
        hb = np.array([(plane >> j) & 1 for j in range(32)], dtype=np.int32)
        assert np.array_equal(got, d * ((lo | (hb << 4)) - 16).astype(np.float32))


def test_quantize_known_answers(oracle):
    # amax 7 -> d = 1 exactly, so codes are round(v) + 8 with halves away from zero.
    v = np.zeros(32, dtype=np.float32)
    v[0], v[1], v[2], v[3], v[16], v[31] = 7.0, -7.0, 2.5, -2.5, 0.49, -3.5
    q = oracle.quantize(Q4, v.reshape(1, 32))
    assert q[:2].tobytes() == np.float16(1.0).tobytes()
    nib = lambda i: (q[2 + i % 16] >> (4 * (i // 16))) & 15
    assert [nib(0), nib(1), nib(2), nib(3), nib(16), nib(31)] == [15, 1, 11, 5, 8, 4]
    # Q8: d = amax / 127 stored as f16, codes against that rounded scale.
    w = np.linspace(-1, 1, 32, dtype=np.float32)
    q8 = oracle.quantize(Q8, w.reshape(1, 32))
    d16 = np.frombuffer(q8[:2].tobytes(), dtype=np.float16)[0]
    assert d16 == np.float16(np.float32(1.0) / np.float32(127.0))
    assert q8[2:].view(np.int8)[0] == -127 and q8[2:].view(np.int8)[-1] == 127
    # Q5: 15 levels either side; the fifth bit goes to the plane.
    v5 = np.zeros(32, dtype=np.float32)
    v5[0], v5[20] = 15.0, -15.0
    q5 = oracle.quantize(Q5, v5.reshape(1, 32))
    plane = int.from_bytes(q5[2:6].tobytes(), "little")
    assert (plane & 1) == 1 and ((plane >> 20) & 1) == 0
    assert q5[6] & 15 == 15 and (q5[6 + 4] >> 4) == 1
    # An all-zero block has scale 0 and mid codes.
    z = oracle.quantize(Q4, np.zeros((1, 32), dtype=np.float32))
    assert z[:2].tobytes() == b"\x00\x00" and set(z[2:].tolist()) == {0x88}


def test_quant_roundtrip_within_tolerance(oracle):
    """src/quant.rs:521-540."""
    row = np.array([((i * 37 % 71) - 35.0) / 10.0 for i in range(128)], dtype=np.float32).reshape(1, 128)
    for dt, tol in [(F32, 1e-6), (F16, 1e-2), (Q8, 3e-2), (Q5, 0.12), (Q4, 0.4)]:
        back = oracle.dequant(dt, oracle.quantize(dt, row), 1, 128)
        assert np.abs(back - row).max() < tol, dt


def test_more_bits_costs_more_and_loses_less(oracle):
    """src/quant.rs:545-577 (Q6 omitted: not a format of this path)."""
    row = np.array([(i / 255.0 - 0.5) * (9.0 if i == 3 else 2.0) for i in range(256)], dtype=np.float32)
    prev = None
    for dt in (Q4, Q5, Q8):
        q = oracle.quantize(dt, row.reshape(1, 256))
        err = np.abs(oracle.dequant(dt, q, 1, 256)[0] - row).max()
        if prev:
            assert q.size > prev[0] and err < prev[1]
        prev = (q.size, err)


def test_every_level_round_trips(oracle):
    """src/quant.rs:581-597."""
    for dt, levels in [(Q4, 15), (Q5, 31), (Q8, 255)]:
        half = levels // 2
        row = np.array([(i % (half + 1)) - half // 2 for i in range(32)], dtype=np.float32).reshape(1, 32)
        back = oracle.dequant(dt, oracle.quantize(dt, row), 1, 32)
        step = np.abs(row).max() / max(half, 1)
        assert np.abs(back - row).max() <= step * 0.75, dt
