"""Pin the CPU oracle's bit layout and packed products.

Golden vectors: the reference's committed fixtures (tests/golden/*.json,
copied from crates/quantibbler-kernels/tests/fixtures/), plus closed forms
and brute force that a plausible mistake (bit order, sign, transposed
operand, wrong accumulator) would fail.
"""
import numpy as np
import pytest

from conftest import load_golden


def test_pack_bits_fixture(orc):
    for rec in load_golden("pack_bits.json"):
        exp = rec["faces"]["numpy-reference"]
        factor = np.array(rec["inputs"]["factor"], dtype=np.int8)
        nb = rec["dtypes"]["n_bits"]
        if "shape" in rec["inputs"]:
            factor = factor.reshape(rec["inputs"]["shape"])
        rows = factor.shape[0] if factor.ndim == 2 else 0
        packed = orc.pack_bits(factor.reshape(rows, nb)) if rows else np.zeros((0, (nb + 7) // 8), np.uint8)
        assert packed.tolist() == np.array(exp["packed"], dtype=np.uint8).reshape(packed.shape).tolist(), rec["scenario"]
        if "unpacked" in exp:
            un = orc.unpack_bits(packed, nb)
            assert un.tolist() == exp["unpacked"], rec["scenario"]
        if "expected_bytes" in exp:
            assert packed.ravel().tolist() == np.array(exp["expected_bytes"]).ravel().tolist()


def test_pack_bits_closed_form(orc):
    # element k alone set to +1: byte k//8 == 2**(k%8), every other byte 0
    # (openspec/specs/qk-kernels/spec.md:40-45)
    n = 37
    for k in range(n):
        f = -np.ones((1, n), np.int8)
        f[0, k] = 1
        p = orc.pack_bits(f)[0]
        want = np.zeros((n + 7) // 8, np.uint8)
        want[k // 8] = 1 << (k % 8)
        assert p.tolist() == want.tolist()


def test_pack_rejects_non_binary_with_reference_text(orc):
    f = np.ones((2, 3), np.int8)
    f[1, 2] = 0
    with pytest.raises(orc.OracleError, match=r"pack_bits expects values in \{-1, \+1\}; got 0 at row 1, column 2"):
        orc.pack_bits(f)


def test_unpack_and_validate_messages(orc):
    with pytest.raises(orc.OracleError, match="packed length 3 does not match 2 rows x 1 bitplanes"):
        orc.unpack_bits(np.zeros(3, np.uint8), 8, n_rows=2)
    with pytest.raises(orc.OracleError, match="n_bits=0 with non-empty packed rows"):
        orc.validate_packed(2, 2, 0)
    assert orc.validate_packed(0, 0, 0) == 0
    # pad bits are ignored by unpack
    assert orc.unpack_bits(np.array([[0xFF, 0xFF]], np.uint8), 9).tolist() == [[1] * 9]


def test_sign_estimate_fixture(orc):
    for rec in load_golden("sign_estimate.json"):
        x = np.array(rec["inputs"]["x"], np.float64)
        assert orc.sign_estimate(x).tolist() == rec["faces"]["numpy-reference"]["signs"]


def test_packed_matvec_fixture_bit_identical(orc):
    for rec in load_golden("packed_matvec.json"):
        p = np.array(rec["inputs"]["packed"], np.uint8)
        v = np.array(rec["inputs"]["vec"], np.float64)
        nb = rec["dtypes"]["n_bits"]
        got = orc.packed_matvec(p, p.shape[0], nb, v)
        assert got.tobytes() == np.array(rec["faces"]["numpy-reference"]["result"]).tobytes()
        if "packed_dirty" in rec["inputs"]:
            pd = np.array(rec["inputs"]["packed_dirty"], np.uint8)
            got = orc.packed_matvec(pd, p.shape[0], nb, v)
            assert got.tobytes() == np.array(rec["faces"]["numpy-reference"]["result_dirty"]).tobytes()


def test_packed_matmul_fixture_bit_identical(orc):
    for rec in load_golden("packed_matmul.json"):
        p = np.array(rec["inputs"]["packed"], np.uint8)
        m = np.array(rec["inputs"]["mat"], np.float64)
        got = orc.packed_matmul(p, p.shape[0], m.shape[0], m, m.shape[1])
        assert got.tobytes() == np.array(rec["faces"]["numpy-reference"]["result"]).tobytes()


def test_dtype_parity_fixture_exact(orc):
    for rec in load_golden("dtype_parity.json"):
        dt = rec["dtypes"]["operand"]
        npd = {"float32": np.float32, "bfloat16": np.uint16}[dt]
        p = np.array(rec["inputs"]["packed"], np.uint8)
        nb = rec["dtypes"]["n_bits"]
        exp = np.array(rec["faces"]["numpy-reference"]["result"], dtype=npd)
        if "vec" in rec["inputs"]:
            got = orc.packed_matvec(p, p.shape[0], nb, np.array(rec["inputs"]["vec"], npd), dt)
        else:
            m = np.array(rec["inputs"]["mat"], dtype=npd)
            got = orc.packed_matmul(p, p.shape[0], nb, m, m.shape[1], dt)
        assert got.tobytes() == exp.reshape(got.shape).tobytes(), rec["scenario"]


def test_bf16_round_to_nearest_even_kats(orc):
    # dtype.rs:179-180: half an 8-bit ulp above 1.0 rounds to 1.0 (even)
    assert orc.f32_to_bf16(np.float32(1 + 2 ** -8)) == 0x3F80
    assert orc.f32_to_bf16(np.float32(1 + 3 * 2 ** -8)) == 0x3F82  # tie -> even (up)
    assert orc.f32_to_bf16(np.float32(1 + 2 ** -8 + 2 ** -20)) == 0x3F81  # above tie
    x = np.random.default_rng(0).standard_normal(4096).astype(np.float32)
    assert np.array_equal(orc.f32_to_bf16(x), orc.f32_to_bf16_fast(x))


@pytest.mark.parametrize("dtype", ["float64", "float32", "bfloat16"])
def test_products_against_brute_force(orc, dtype):
    rng = np.random.default_rng(11)
    n_rows, n_bits, k = 23, 77, 5
    signs = rng.choice([-1, 1], size=(n_rows, n_bits)).astype(np.int8)
    packed = orc.pack_bits(signs)
    vals = rng.standard_normal((n_bits, k))
    if dtype == "bfloat16":
        op = orc.f32_to_bf16(vals.astype(np.float32))
        dense = orc.bf16_to_f32(op).astype(np.float64)
    else:
        op = vals.astype(dtype)
        dense = op.astype(np.float64)
    exact = signs.astype(np.float64) @ dense
    mv = orc.packed_matvec(packed, n_rows, n_bits, op[:, 0].copy(), dtype)
    mm = orc.packed_matmul(packed, n_rows, n_bits, op, k, dtype)
    scale = np.abs(dense).sum(axis=0)
    tol = {"float64": 1e-14, "float32": 1e-6, "bfloat16": 1e-2}[dtype]
    f = orc.bf16_to_f32 if dtype == "bfloat16" else (lambda a: a)
    assert np.all(np.abs(f(mv).astype(np.float64) - exact[:, 0]) <= tol * scale[0])
    assert np.all(np.abs(f(mm).astype(np.float64) - exact) <= tol * scale[None, :])
    # a wrong sign convention or transposed bit order would be O(1) off
    assert np.allclose(f(mm).astype(np.float64), exact, rtol=0, atol=0.05 * scale.max())


def test_matmul_degenerate_and_n_cols_contract(orc):
    p = np.zeros((2, 1), np.uint8)
    assert orc.packed_matmul(p, 2, 8, np.zeros(0), 0).shape == (2, 0)
    with pytest.raises(orc.OracleError, match="mat length 7 is not a multiple of n_bits 8"):
        orc.packed_matmul(p, 2, 8, np.zeros(7), 1)
    # n_cols participates in the addressing (core.rs:302-316)
    m = np.arange(16, dtype=np.float64)
    got = orc.packed_matmul(np.array([[0xFF]], np.uint8), 1, 8, m, 2)
    assert got.tolist() == [[sum(m[t * 2] for t in range(8)), sum(m[t * 2 + 1] for t in range(8))]]


def test_fast_face_backward_error_and_repeatability(orc):
    # fast_cpu_parity.rs:47-75: backward error <= 1e-12 sum|v|, bit identity
    rng = np.random.default_rng(5)
    for n_rows, n_bits in [(1, 1), (257, 73), (1024, 137), (64, 8)]:
        signs = rng.choice([-1, 1], size=(n_rows, n_bits)).astype(np.int8)
        packed = orc.pack_bits(signs)
        v = rng.standard_normal(n_bits)
        seq = orc.packed_matvec(packed, n_rows, n_bits, v)
        runs = [orc.fast_packed_matvec(packed, n_rows, n_bits, v, threads=t) for t in (1, 3, 8)]
        for r in runs[1:]:
            assert r.tobytes() == runs[0].tobytes()
        assert np.all(np.abs(runs[0] - seq) <= 1e-12 * np.abs(v).sum())
        m = rng.standard_normal((n_bits, 3))
        assert orc.fast_packed_matmul(packed, n_rows, n_bits, m, 3).tobytes() == \
            orc.packed_matmul(packed, n_rows, n_bits, m, 3).tobytes()


def test_head_logits_pins(orc):
    """engine/mod.rs:781-800 Engine::logits, pinned without retyping it:
    the summation order (2^24 + 1 - 2^24 is 0 only left to right), separate
    multiply and add (a case an FMA rounds differently), one-hot rows (a
    column of the head exactly), and integer inputs (exact int64 products)."""
    h = np.array([[2.0 ** 24, 1.0, -2.0 ** 24], [2.0 ** 24, -2.0 ** 24, 1.0]], np.float32)
    assert orc.head_logits(h, np.ones(3, np.float32)).tolist() == [0.0, 1.0]
    # acc = -0x1.00060ap+0 after t = 0, then + h*w: 0x1.97ap-12 with the
    # product rounded first, 0x1.97af7ep-12 fused
    hh = np.array([[float.fromhex("-0x1.00060ap+0"), float.fromhex("0x1.00106p+0")]], np.float32)
    x = np.array([1.0, float.fromhex("0x1.000f24p+0")], np.float32)
    assert orc.head_logits(hh, x)[0] == np.float32(float.fromhex("0x1.97ap-12"))
    rng = np.random.default_rng(4)
    head = rng.standard_normal((37, 19)).astype(np.float32)
    for t in (0, 7, 18):
        e = np.zeros(19, np.float32)
        e[t] = 1.0
        assert orc.head_logits(head, e).tobytes() == head[:, t].tobytes()
    hi = rng.integers(-8, 9, (50, 33)).astype(np.float32)
    xi = rng.integers(-8, 9, (3, 33)).astype(np.float32)
    want = (xi.astype(np.int64) @ hi.astype(np.int64).T).astype(np.float32)
    assert orc.head_logits(hi, xi).tobytes() == want.tobytes()
