"""Pin the attention oracles.

* exact tiled attention: attention_tiled.json (9 cases) and the dense
  softmax closed form;
* the [SA] s4 reference scheme, f64 NumPy semantics: attention_sage.json
  quantized-reference.out (10 cases, seeds 9100-9109);
* the same scheme in the device face's f32 order: within the device gate of
  crates/quantibbler-kernels/tests/gpu_attention_sage.rs:35-46 (two-part
  rel 1e-4, band 1e-1) and inside the reference's measured quality envelope;
* orc_expf against libm exp;
* the block-scaled scheme (no reference implementation: parity with the
  reference UNPINNED) against exact attention quality and its quantizer
  invariants.
"""
import math

import numpy as np
import pytest

from conftest import load_golden

RTOL, BAND = 1e-4, 1e-1
COS_MIN, RL1_MAX, SLACK = 0.999, 0.02, 1e-3


def shaped(rec, name, kind):
    s = rec["shape"]
    heads = s["n_heads"] if kind == "q" else s["n_kv_heads"]
    last = s["val_dim"] if kind == "v" else s["head_dim"]
    return np.array(rec["inputs"][name], np.float32).reshape(s["batch"], heads, s["seq"], last)


def two_part_gate(actual, expected, row_len):
    """gpu_attention_sage.rs:98-143."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    norm = max(np.abs(a).max(), np.abs(e).max())
    assert np.isfinite(norm) and norm > 0
    assert np.abs(a - e).max() <= RTOL * norm
    rows_e = e.reshape(-1, row_len)
    rows_a = a.reshape(-1, row_len)
    rmax = np.abs(rows_e).max(axis=1, keepdims=True)
    m = (np.abs(rows_e) >= BAND * rmax) & (np.abs(rows_e) > 0)
    worst = (np.abs(rows_a - rows_e)[m] / np.abs(rows_e)[m]).max() if m.any() else 0.0
    assert worst <= RTOL, worst
    return worst


def metrics(actual, exact):
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(exact, np.float64).ravel()
    cos = float(a @ e / (np.linalg.norm(a) * np.linalg.norm(e)))
    rl1 = float(np.abs(a - e).sum() / np.abs(e).sum())
    return cos, rl1


def dense_attention(q, k, v, causal):
    b, h, s, d = q.shape
    g = h // k.shape[1]
    kk = np.repeat(k, g, axis=1)
    vv = np.repeat(v, g, axis=1)
    sc = (q @ kk.swapaxes(-1, -2)) / math.sqrt(d)
    if causal:
        sc = np.where(np.triu(np.ones((s, s), bool), 1), -np.inf, sc)
    sc = sc - sc.max(axis=-1, keepdims=True)
    p = np.exp(sc)
    return (p / p.sum(axis=-1, keepdims=True)) @ vv


def test_attention_tiled_fixture(orc):
    for rec in load_golden("attention_tiled.json"):
        q, k, v = (shaped(rec, n, t).astype(np.float64) for n, t in
                   (("query", "q"), ("key", "k"), ("value", "v")))
        out = orc.attention_tiled(q, k, v, causal=rec["causal"])
        exp = np.array(rec["faces"]["numpy-reference"]["out"])
        assert np.abs(out.ravel() - exp).max() <= 1e-12 * np.abs(exp).max()
        dense = dense_attention(q, k, v, rec["causal"])
        assert np.abs(out - dense).max() <= 1e-12 * np.abs(dense).max()


def test_attention_tiled_block_invariance_and_lse(orc):
    rng = np.random.default_rng(1)
    q, k, v = rng.standard_normal((1, 4, 37, 8)), rng.standard_normal((1, 2, 37, 8)), rng.standard_normal((1, 2, 37, 8))
    ref, lse = orc.attention_tiled(q, k, v, causal=True, block_size=64, return_lse=True)
    for bs in (1, 5, 16):
        assert np.abs(orc.attention_tiled(q, k, v, causal=True, block_size=bs) - ref).max() < 1e-13
    sc = (q @ np.repeat(k, 2, 1).swapaxes(-1, -2)) / math.sqrt(8)
    sc = np.where(np.triu(np.ones((37, 37), bool), 1), -np.inf, sc)
    m = sc.max(-1)
    assert np.abs(lse - (m + np.log(np.exp(sc - m[..., None]).sum(-1)))).max() < 1e-12


def test_attention_sage_np_fixture(orc):
    for rec in load_golden("attention_sage.json"):
        q, k, v = (shaped(rec, n, t).astype(np.float64) for n, t in
                   (("query", "q"), ("key", "k"), ("value", "v")))
        out = orc.attention_sage_np(q, k, v, causal=rec["causal"], block_size=rec["block_size"])
        exp = np.array(rec["faces"]["quantized-reference"]["out"])
        assert np.abs(out.ravel() - exp).max() <= 1e-12 * np.abs(exp).max(), rec["seed"]


def test_attention_sage_dev_f32_within_device_gate(orc):
    for rec in load_golden("attention_sage.json"):
        q, k, v = (shaped(rec, n, t) for n, t in (("query", "q"), ("key", "k"), ("value", "v")))
        out = orc.attention_sage_dev(q, k, v, causal=rec["causal"], block_size=rec["block_size"])
        two_part_gate(out, rec["faces"]["quantized-reference"]["out"], rec["shape"]["val_dim"])
        cos, rl1 = metrics(out, rec["faces"]["exact"]["out"])
        ref = rec["reference_metrics"]
        assert cos >= COS_MIN and rl1 <= RL1_MAX
        assert cos >= ref["cosine"] - SLACK and rl1 <= ref["relative_l1"] + SLACK


def test_sage_reference_invariants(orc):
    # tests/test_attention_sage.py:299-763 (gamma shift invariance, block-1
    # exactness, exact-zero causal future)
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 2, 12, 8))
    k = rng.standard_normal((1, 1, 12, 8))
    v = rng.standard_normal((1, 1, 12, 8))
    base = orc.attention_sage_np(q, k, v, causal=True, block_size=4)
    shifted = orc.attention_sage_np(q, k + rng.standard_normal(8) * 5.0, v, causal=True, block_size=4)
    assert np.abs(base - shifted).max() <= 1e-12 * np.abs(base).max()
    # block 1: gamma == 0, codes 0, the shift restores exact keys; only P and V
    # quantisation remain, so it stays close to exact
    one = orc.attention_sage_np(q, k, v, causal=True, block_size=1)
    cos, rl1 = metrics(one, dense_attention(q, k, v, True))
    assert cos > 0.999 and rl1 < 0.02
    # causal: changing future keys/values does not change earlier rows
    k2, v2 = k.copy(), v.copy()
    k2[..., 8:, :] += 3.0
    v2[..., 8:, :] -= 2.0
    a = orc.attention_sage_dev(q.astype(np.float32), k2.astype(np.float32), v2.astype(np.float32), True, 4)
    b = orc.attention_sage_dev(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), True, 4)
    assert np.array_equal(a[..., :8, :], b[..., :8, :])


def test_expf_accuracy(orc):
    xs = np.concatenate([np.linspace(-100, 0, 20001), np.linspace(-1, 1, 2001), [0.0, -0.0, -1e-30]])
    for x in xs:
        got = orc.expf(float(np.float32(x)))
        want = math.exp(float(np.float32(x)))
        if want < 1.2e-38:
            assert abs(got - want) <= 2e-45 * 4
        else:
            assert abs(got - want) <= 2.5 * np.spacing(np.float32(want)), (x, got, want)
    assert orc.expf(0.0) == 1.0 and orc.expf(-200.0) == 0.0


def _blk_inputs(rng, b, h, hk, s, d=128, offset_std=2.0):
    q = rng.standard_normal((b, h, s, d)).astype(np.float32)
    k = (rng.standard_normal((b, hk, s, d)) + offset_std * rng.standard_normal((b, hk, 1, d))).astype(np.float32)
    v = rng.standard_normal((b, hk, s, d)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("causal", [True, False])
def test_sage_blk_quality_against_exact(orc, causal):
    rng = np.random.default_rng(9200)
    q, k, v = _blk_inputs(rng, 1, 4, 2, 200)
    qb, kb, vb = (orc.f32_to_bf16_fast(a) for a in (q, k, v))
    out, st = orc.attention_sage_blk(qb, kb, vb, causal=causal, stages=True)
    exact = dense_attention(*(orc.bf16_to_f32(a).astype(np.float64) for a in (qb, kb, vb)), causal)
    cos, rl1 = metrics(out, exact)
    assert cos >= COS_MIN and rl1 <= RL1_MAX, (cos, rl1)
    # quantiser invariants: mean, smoothing, block scales, code ranges
    kf = orc.bf16_to_f32(kb).astype(np.float64)
    assert np.abs(st["kmean"] - kf.mean(axis=2)).max() < 1e-5
    g = kf - st["kmean"][:, :, None, :]
    for blk in range(st["kscale"].shape[2]):
        sl = slice(64 * blk, min(64 * blk + 64, 200))
        peak = np.abs(g[:, :, sl, :]).max(axis=(2, 3))
        assert np.allclose(st["kscale"][:, :, blk], peak / 127, rtol=1e-5)
        deq = st["khat"][:, :, sl, :] * st["kscale"][:, :, blk][..., None, None]
        assert np.abs(deq - g[:, :, sl, :]).max() <= 0.5001 * st["kscale"][:, :, blk].max() + 1e-5
    assert np.abs(st["qhat"]).max() == 127 and np.abs(st["khat"]).max() == 127


def test_sage_blk_mean_shift_invariance(orc):
    # a per-channel offset added to every key changes nothing but the mean
    rng = np.random.default_rng(9201)
    q, k, v = _blk_inputs(rng, 1, 2, 1, 128, offset_std=0.0)
    off = (4.0 * rng.standard_normal(128)).astype(np.float32)
    qb, vb = orc.f32_to_bf16_fast(q), orc.f32_to_bf16_fast(v)
    kb = orc.f32_to_bf16_fast(np.round(k * 8) / 8)
    kb2 = orc.f32_to_bf16_fast(orc.bf16_to_f32(kb) + np.round(off * 8) / 8)
    o1 = orc.attention_sage_blk(qb, kb, vb, causal=True)
    o2 = orc.attention_sage_blk(qb, kb2, vb, causal=True)
    cos, rl1 = metrics(o1, o2)
    assert cos > 0.9999 and rl1 < 5e-3
