"""Pins of the oracle's decoder-block pieces (engine/mod.rs:837-852,
:1154-1187) against what the mathematics fixes: RoPE at position 0 is the
identity, at other positions it is the rotation of each (i, i + hd/2) pair
by pos * theta^(-2i/hd) (checked against complex multiplication in f64) and
keeps each pair's norm; the bf16 RMSNorm of a constant vector is
c / sqrt(c^2 + eps), and with eps = 0 it is invariant under scaling by a
power of two (bit for bit: every step scales exactly)."""
import math

import numpy as np


def test_rope_rotate_pins(orc):
    rng = np.random.default_rng(3)
    v = rng.standard_normal(3 * 8).astype(np.float32)
    assert orc.rope_rotate(v, 8, 0, 10000.0).tobytes() == v.tobytes()
    for pos in (1, 7, 1000):
        got = orc.rope_rotate(v, 8, pos, 10000.0)
        for base in range(0, len(v), 8):
            for i in range(4):
                ang = pos * math.pow(10000.0, -(2.0 * i) / 8)
                z = complex(float(v[base + i]), float(v[base + 4 + i])) * complex(math.cos(ang), math.sin(ang))
                assert abs(got[base + i] - z.real) <= 1e-5 * (1 + abs(z))
                assert abs(got[base + 4 + i] - z.imag) <= 1e-5 * (1 + abs(z))
                n0 = math.hypot(v[base + i], v[base + 4 + i])
                n1 = math.hypot(got[base + i], got[base + 4 + i])
                assert abs(n0 - n1) <= 1e-5 * (1 + n0)


def test_rms_norm_bf16_pins(orc):
    d = 64
    for c, eps in ((1.5, 1e-5), (-0.375, 1e-6), (3.0, 0.0)):
        x = np.full(d, c, np.float32)
        got = orc.rms_norm_bf16(x, np.ones(d, np.float32), eps)
        want = c / math.sqrt(c * c + eps)
        assert np.all(np.abs(got - want) <= 2 ** -8 * abs(want))
    rng = np.random.default_rng(5)
    x = orc.bf16_to_f32(orc.f32_to_bf16_fast(rng.standard_normal(d).astype(np.float32)))
    w = rng.standard_normal(d).astype(np.float32)
    base = orc.rms_norm_bf16(x, w, 0.0)
    for k in (0.25, 2.0, 64.0):
        assert orc.rms_norm_bf16((x * np.float32(k)).astype(np.float32), w, 0.0).tobytes() == base.tobytes()
    # a planted mistake (weights applied before the normalisation's rounding
    # of the operand would not change this, but a missing square root would)
    bad = orc.bf16_to_f32(orc.f32_to_bf16_fast((x / np.float32(np.mean(x * x))) * w))
    assert bad.tobytes() != base.tobytes()
