"""joint_itq (core.rs:318-424) through the PyO3-named face, host code in
libqbk, against the reference's joint_itq.json fixture (4 records: converged,
fixed max_iter, seed determinism, product preservation): u_t, v_t byte-equal
and n_iter / converged equal to the numpy-reference face, as
crates/quantibbler-kernels/tests/parity.rs:344-406 requires of the Rust
face.  Runs on the CPU (no device involved)."""
import numpy as np
import pytest

from conftest import load_golden


def test_joint_itq_fixture_exact():
    from quantibbler_amd import kernels as K

    for rec in load_golden("joint_itq.json"):
        u = np.array(rec["inputs"]["u_hat"], np.float64)
        v = np.array(rec["inputs"]["v_hat"], np.float64)
        kw = rec["inputs"]["kwargs"]
        ut, vt, n_iter, conv = K.joint_itq(u, v, max_iter=kw["max_iter"], tol=kw["tol"], seed=kw["seed"])
        np_face = rec["faces"]["numpy-reference"]
        assert n_iter == np_face["n_iter"], rec["scenario"]
        assert conv == np_face["converged"], rec["scenario"]
        assert ut.tolist() == np.array(np_face["u_t"], np.int8).reshape(ut.shape).tolist(), rec["scenario"]
        assert vt.tolist() == np.array(np_face["v_t"], np.int8).reshape(vt.shape).tolist(), rec["scenario"]
        if "repeat_u_t" in np_face:
            u2, v2, n2, _ = K.joint_itq(u, v, max_iter=kw["max_iter"], tol=kw["tol"], seed=kw["seed"])
            assert u2.tolist() == ut.tolist() and v2.tolist() == vt.tolist() and n2 == n_iter


def test_joint_itq_properties_and_errors():
    from quantibbler_amd import KernelError
    from quantibbler_amd import kernels as K

    rng = np.random.default_rng(3)
    u, v = rng.standard_normal((40, 12)), rng.standard_normal((30, 12))
    ut, vt, n_iter, conv = K.joint_itq(u, v, seed=7)
    assert set(np.unique(ut)) <= {-1, 1} and set(np.unique(vt)) <= {-1, 1}
    assert 1 <= n_iter <= 50
    # a rotated input: Z R for an orthogonal R gives the same codes up to the rotation the solver finds,
    # so the objective ||B - Z R||_F it reaches is the same (fixed-point property)
    _, _, n_fixed, c_fixed = K.joint_itq(u, v, max_iter=50, tol=0.0, seed=7)
    assert n_fixed == 50 and c_fixed is False
    with pytest.raises(KernelError, match="joint_itq rank mismatch: u_hat r=12, v_hat r=11"):
        K.joint_itq(u, v[:, :11])
    with pytest.raises(KernelError, match="joint_itq expects non-empty factors"):
        K.joint_itq(np.zeros((3, 0)), np.zeros((2, 0)))
