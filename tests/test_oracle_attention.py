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


# ---- block-scaled scheme: closed forms a plausible mistake would fail --------

def _f32(a):
    return np.asarray(a, np.float32)


def _codes(x, peak):
    """INT8 codes of x at one block's peak, in the f32 order the scheme fixes:
    invs = 127 / peak, rint(x * invs) half-even, clamped to +-127."""
    invs = np.float32(127.0) / np.float32(peak) if peak > 0 else np.float32(0.0)
    return np.clip(np.rint(_f32(x) * invs), -127, 127).astype(np.int8)


@pytest.mark.parametrize("s", [64, 200])
def test_sage_blk_q_and_k_codes_closed_form(orc, s):
    """Q: one scale per 64-token block per head, taken over exactly tokens
    64b .. 64b+63 of x = q * (1/sqrt(d)) (f32), scale = peak / 127, codes by
    round-half-even.  K: the same over g = k - mean.  A per-token scale, a
    block window off by one token, or truncating codes all fail here."""
    rng = np.random.default_rng(9300 + s)
    q, k, v = _blk_inputs(rng, 1, 4, 2, s)
    # vary each token's magnitude so that a per-token scale would differ
    q *= np.exp(rng.standard_normal((1, 4, s, 1))).astype(np.float32)
    qb, kb, vb = (orc.f32_to_bf16_fast(a) for a in (q, k, v))
    _, st = orc.attention_sage_blk(qb, kb, vb, causal=True, stages=True)
    inv_sqrt_d = np.float32(1.0) / np.sqrt(np.float32(128.0))
    x = _f32(orc.bf16_to_f32(qb)) * inv_sqrt_d
    g = _f32(orc.bf16_to_f32(kb)) - st["kmean"][:, :, None, :]
    nblk = (s + 63) // 64
    for h in range(4):
        for blk in range(nblk):
            sl = slice(64 * blk, min(64 * blk + 64, s))
            peak = np.abs(x[0, h, sl]).max()
            assert st["qscale"][0, h, blk] == np.float32(peak) / np.float32(127.0)
            assert np.array_equal(st["qhat"][0, h, sl], _codes(x[0, h, sl], peak)), (h, blk)
    for hk in range(2):
        for blk in range(nblk):
            sl = slice(64 * blk, min(64 * blk + 64, s))
            peak = np.abs(g[0, hk, sl]).max()
            assert st["kscale"][0, hk, blk] == np.float32(peak) / np.float32(127.0)
            assert np.array_equal(st["khat"][0, hk, sl], _codes(g[0, hk, sl], peak)), (hk, blk)
    # half-even: a code from an exact .5 rounds to the even neighbour
    assert _codes(np.array([0.5, 1.5, 2.5, -0.5], np.float32), 127.0).tolist() == [0, 2, 2, 0]


def test_sage_blk_identical_keys_give_the_mean_of_v(orc):
    """Every key equal: K - mean is zero, so every score is 0, p = 1 for every
    key in the window, and row i's output is the mean of V over keys 0..i
    (causal) -- V as the fp16 values P.V multiplies."""
    rng = np.random.default_rng(9310)
    s = 130
    q = rng.standard_normal((1, 2, s, 128)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 1, 1, 128)).astype(np.float32), s, axis=2)
    v = rng.standard_normal((1, 1, s, 128)).astype(np.float32)
    qb, kb, vb = (orc.f32_to_bf16_fast(a) for a in (q, k, v))
    out = orc.attention_sage_blk(qb, kb, vb, causal=True).astype(np.float64)
    vf = orc.bf16_to_f32(vb).astype(np.float16).astype(np.float64)[0, 0]
    want = np.cumsum(vf, axis=0) / np.arange(1, s + 1)[:, None]
    for h in range(2):
        assert np.abs(out[0, h] - want).max() <= 1e-6 * np.abs(vf).max(), h
    out_nc = orc.attention_sage_blk(qb, kb, vb, causal=False).astype(np.float64)
    assert np.abs(out_nc[0, 0] - vf.mean(axis=0)[None, :]).max() <= 1e-6 * np.abs(vf).max()


def test_sage_blk_one_hot_softmax_returns_that_value_row(orc):
    """One key whose score exceeds every other by more than 150 (log2 units):
    every other p underflows to zero in exp2, so the output row is exactly
    that key's V row (its fp16 value; bf16 V values are fp16-exact here)."""
    s, star = 96, 70
    q = np.zeros((1, 1, s, 128), np.float32)
    q[..., 0] = 64.0
    k = np.zeros((1, 1, s, 128), np.float32)
    k[0, 0, :, 0] = -1.0
    k[0, 0, star, 0] = 60.0
    rng = np.random.default_rng(9320)
    v = rng.standard_normal((1, 1, s, 128)).astype(np.float32)
    qb, kb, vb = (orc.f32_to_bf16_fast(a) for a in (q, k, v))
    out = orc.attention_sage_blk(qb, kb, vb, causal=False)
    vf = orc.bf16_to_f32(vb)[0, 0]
    assert np.array_equal(out[0, 0], np.broadcast_to(vf[star], (s, 128)))
    # causal: rows from the star on see it; rows of the first key block
    # (whose keys all share one code and one scale) weigh keys 0..i alike
    outc = orc.attention_sage_blk(qb, kb, vb, causal=True).astype(np.float64)
    assert np.array_equal(outc[0, 0, star:], np.broadcast_to(vf[star], (s - star, 128)).astype(np.float64))
    want = np.cumsum(vf.astype(np.float64), axis=0) / np.arange(1, s + 1)[:, None]
    assert np.abs(outc[0, 0, :64] - want[:64]).max() <= 1e-6


def test_sage_blk_p_is_fp16_and_ell_unquantised(orc):
    """Two keys at scores +s0 and -s0 (codes +-127, mean 0): p0 = 1,
    p1 = 2^(-2 s0).  With V = (0, 1) on one channel the output is
    fp16(p1) / (1 + p1): P.V multiplies the fp16 P, the row sum l adds the
    f32 p.  A bf16 P, an f32 P or an l over the rounded P each miss it."""
    q = np.zeros((1, 1, 2, 128), np.float32)
    q[..., 0] = 4.0
    k = np.zeros((1, 1, 2, 128), np.float32)
    k[0, 0, 0, 0], k[0, 0, 1, 0] = 1.0, -1.0
    v = np.zeros((1, 1, 2, 128), np.float32)
    v[0, 0, 1, 5] = 1.0
    qb, kb, vb = (orc.f32_to_bf16_fast(a) for a in (q, k, v))
    out, st = orc.attention_sage_blk(qb, kb, vb, causal=False, stages=True)
    assert st["khat"][0, 0, :, 0].tolist() == [127, -127] and st["qhat"][0, 0, :, 0].tolist() == [127, 127]
    cs = np.float32(np.float32(st["qscale"][0, 0, 0] * st["kscale"][0, 0, 0]) * np.float32(1.4426950408889634))
    s0 = np.float32(np.float32(127 * 127) * cs)
    p1 = float(np.exp2(np.float64(np.float32(-s0) - s0)))
    assert 0.3 < p1 < 0.7
    want = float(np.float16(p1)) / (1.0 + p1)
    got = float(out[0, 0, 0, 5])
    assert abs(got - want) <= 4e-7 * want, (got, want)
    bf16_p = float(orc.bf16_to_f32(orc.f32_to_bf16(np.array([p1], np.float32)))[0])
    assert abs(bf16_p / (1 + p1) - want) > 100 * 4e-7 * want
    assert abs(p1 / (1 + p1) - want) > 100 * 4e-7 * want
    assert abs(float(np.float16(p1)) / (1 + float(np.float16(p1))) - want) > 100 * 4e-7 * want
