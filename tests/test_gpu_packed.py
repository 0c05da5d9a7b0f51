"""GPU parity: the packed products (gpu.rs:116-185, dispatch.rs:81-109) through
the C ABI against the oracle.  The device sums each output in element order,
so every dtype is expected bit-identical (gpu_parity.rs:50-93 asks rel 1e-12
and run-to-run bit identity for f64)."""
import numpy as np
import pytest

from conftest import load_golden, same

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def say(*a):
    print(*a, flush=True)


def test_fixtures_bit_identical(ctx, orc):
    for rec in load_golden("packed_matvec.json"):
        p = np.array(rec["inputs"]["packed"], np.uint8)
        v = np.array(rec["inputs"]["vec"], np.float64)
        say("packed_matvec fixture", rec["scenario"])
        got = ctx.packed_matvec(p, p.shape[0], rec["dtypes"]["n_bits"], v)
        same(got, np.array(rec["faces"]["numpy-reference"]["result"]))
        if "packed_dirty" in rec["inputs"]:
            pd = np.array(rec["inputs"]["packed_dirty"], np.uint8)
            got = ctx.packed_matvec(pd, p.shape[0], rec["dtypes"]["n_bits"], v)
            same(got, np.array(rec["faces"]["numpy-reference"]["result_dirty"]))
    for rec in load_golden("packed_matmul.json"):
        p = np.array(rec["inputs"]["packed"], np.uint8)
        m = np.array(rec["inputs"]["mat"], np.float64)
        say("packed_matmul fixture", rec["scenario"])
        got = ctx.packed_matmul(p, p.shape[0], m.shape[0], m, m.shape[1])
        same(got, np.array(rec["faces"]["numpy-reference"]["result"]))
    for rec in load_golden("dtype_parity.json"):
        dt = rec["dtypes"]["operand"]
        npd = {"float32": np.float32, "bfloat16": np.uint16}[dt]
        p = np.array(rec["inputs"]["packed"], np.uint8)
        nb = rec["dtypes"]["n_bits"]
        exp = np.array(rec["faces"]["numpy-reference"]["result"], npd)
        say("dtype fixture", rec["scenario"])
        if "vec" in rec["inputs"]:
            got = ctx.packed_matvec(p, p.shape[0], nb, np.array(rec["inputs"]["vec"], npd), dt)
        else:
            m = np.array(rec["inputs"]["mat"], npd)
            got = ctx.packed_matmul(p, p.shape[0], nb, m, m.shape[1], dt)
        same(got, exp.reshape(got.shape))


@pytest.mark.parametrize("dtype", ["float64", "float32", "bfloat16"])
@pytest.mark.parametrize("n_rows,n_bits", [(257, 73), (1, 1), (64, 8), (1024, 4096), (3, 1733)])
def test_random_bit_identical_and_repeatable(ctx, orc, dtype, n_rows, n_bits):
    say("packed products", dtype, n_rows, n_bits)
    rng = np.random.default_rng(n_rows * 7 + n_bits)
    packed = orc.pack_bits(rng.choice([-1, 1], (n_rows, n_bits)).astype(np.int8))
    vals = rng.standard_normal((n_bits, 3))
    op = orc.f32_to_bf16_fast(vals.astype(np.float32)) if dtype == "bfloat16" else vals.astype(dtype)
    v = np.ascontiguousarray(op[:, 0])
    want = orc.packed_matvec(packed, n_rows, n_bits, v, dtype)
    g1 = ctx.packed_matvec(packed, n_rows, n_bits, v, dtype)
    g2 = ctx.packed_matvec(packed, n_rows, n_bits, v, dtype)
    same(g1, g2)
    same(g1, want)
    if n_rows * n_bits <= 300000:
        wm = orc.packed_matmul(packed, n_rows, n_bits, op, 3, dtype)
        gm = ctx.packed_matmul(packed, n_rows, n_bits, op, 3, dtype)
        same(gm, wm)


def test_degenerate_shapes_and_errors(ctx, orc):
    from quantibbler_amd import KernelError

    say("degenerate shapes")
    p = orc.pack_bits(np.array([[1]], np.int8))
    assert ctx.packed_matvec(p, 1, 1, np.array([3.5]))[0] == 3.5
    assert ctx.packed_matvec(np.zeros(0, np.uint8), 0, 8, np.ones(8)).size == 0
    with pytest.raises(KernelError) as e:
        ctx.packed_matvec(p, 1, 9, np.ones(9))
    with pytest.raises(orc.OracleError) as o:
        orc.packed_matvec(p, 1, 9, np.ones(9))
    assert str(e.value) == str(o.value)
    assert ctx.packed_matmul(np.zeros((2, 1), np.uint8), 2, 8, np.zeros(0), 0).shape == (2, 0)


def test_pyo3_face_on_gpu(orc):
    from quantibbler_amd import kernels as K

    say("pyo3-named face")
    rng = np.random.default_rng(8)
    f = rng.choice([-1, 1], (6, 13)).astype(np.int8)
    p = K.pack_bits(f)
    v = rng.standard_normal(13)
    same(K.packed_matvec(p, 13, v), orc.packed_matvec(p, 6, 13, v))
    m = rng.standard_normal((13, 4))
    same(K.packed_matmul(p, 13, m), orc.packed_matmul(p, 6, 13, m, 4))
    vb = orc.f32_to_bf16_fast(v.astype(np.float32))
    same(K.packed_matvec_dtype(p, 13, vb, "bfloat16"), orc.packed_matvec(p, 6, 13, vb, "bfloat16"))


def test_host_bit_layout_on_the_gpu_box(orc):
    """core.rs:129-189 pack_bits / unpack_bits and sign_estimate through the
    product library, in the GPU job: byte-identical to the reference's
    pack_bits.json records (including the 16x16 bit-order record and the
    empty shapes) and sign_estimate.json, and to the oracle on random shapes."""
    from conftest import load_golden

    from quantibbler_amd import kernels as K

    say("host bit layout (A1/A2) vs fixtures")
    for rec in load_golden("pack_bits.json"):
        exp = rec["faces"]["numpy-reference"]
        nb = rec["dtypes"]["n_bits"]
        factor = np.array(rec["inputs"]["factor"], dtype=np.int8)
        if "shape" in rec["inputs"]:
            factor = factor.reshape(rec["inputs"]["shape"])
        rows = factor.shape[0] if factor.ndim == 2 else 0
        f = factor.reshape(rows, nb)
        p = K.pack_bits(f) if rows else np.zeros((0, (nb + 7) // 8), np.uint8)
        assert p.tolist() == np.array(exp["packed"], np.uint8).reshape(p.shape).tolist(), rec["scenario"]
        assert p.tobytes() == orc.pack_bits(f).tobytes() if rows else True
        if "unpacked" in exp:
            assert K.unpack_bits(p, nb, "int8").tolist() == exp["unpacked"], rec["scenario"]
        if "expected_bytes" in exp:
            assert p.ravel().tolist() == np.array(exp["expected_bytes"]).ravel().tolist()
    for rec in load_golden("sign_estimate.json"):
        x = np.array(rec["inputs"]["x"], np.float64)
        assert K.sign_estimate(x).ravel().tolist() == rec["faces"]["numpy-reference"]["signs"], rec["scenario"]
    rng = np.random.default_rng(22)
    for rows, cols in [(5, 11), (3, 64), (7, 1), (1, 129), (33, 1000)]:
        f = rng.choice([-1, 1], (rows, cols)).astype(np.int8)
        p = K.pack_bits(f)
        assert p.tobytes() == orc.pack_bits(f).tobytes()
        assert K.unpack_bits(p, cols, "float64").tolist() == f.astype(np.float64).tolist()
