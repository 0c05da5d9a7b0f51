"""Pins of the oracle's decoder-block pieces (engine/mod.rs:837-941,
:1154-1187, :1399-1402) against what the mathematics fixes.

* RoPE at position 0 is the identity; at other positions it rotates each
  (i, i + hd/2) pair by pos * theta^(-2i/hd) (checked against complex
  multiplication in f64) and keeps each pair's norm.
* The bf16 RMSNorm of a constant vector is c / sqrt(c^2 + eps); with eps = 0
  it is invariant under scaling by a power of two, bit for bit.
* The one-pass prefill (block_prefill = prefill_qkv, prefill_attention,
  prefill_mlp), which the reference does not have -- it runs the block token
  by token (engine/mod.rs:1399-1402) -- is pinned stage by stage:
  - its cache rows are bit-identical to the ones block_step writes at each
    position for the same input rows (block_step is pinned by the reference's
    HF goldens, tests/test_oracle_trunk.py);
  - its q rows match the dense f64 block's (norm, projection, per-head norm,
    RoPE at position t) within bf16 serving's rounding;
  - with q = 0 every block-scaled score is 0, so the attention is the causal
    mean of fp16 V: on integer V rows (every sum exact in f32) each output is
    bf16(f32(sum / count)), compared bit for bit;
  - with the q projection zeroed, the whole block's output rows match a dense
    f64 evaluation of the block with that attention;
  - with real q, the attention rows are within the SageAttention quality gate
    of exact f64 attention over the same rows.
  Planted mistakes -- RoPE at t + 1, the attention output not rounded to bf16
  before o, a head-major operand formed without its transpose -- each fail
  at least one of these.
"""
import math

import numpy as np
import pytest

D, H, HK, HD, FFN = 64, 4, 2, 16, 96
THETA, EPS = 10000.0, 1e-6


def test_rope_pins(orc):
    rng = np.random.default_rng(3)
    v = rng.standard_normal(3 * 8).astype(np.float32)
    assert orc.rope(v, 8, 0, 10000.0).tobytes() == v.tobytes()
    for pos in (1, 7, 1000):
        got = orc.rope(v, 8, pos, 10000.0)
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
        got = orc.norm_apply(x, np.ones(d, np.float32), eps, "bf16")
        want = c / math.sqrt(c * c + eps)
        assert np.all(np.abs(got - want) <= 2 ** -8 * abs(want))
    rng = np.random.default_rng(5)
    x = orc.bf16_round(rng.standard_normal(d).astype(np.float32))
    w = rng.standard_normal(d).astype(np.float32)
    base = orc.norm_apply(x, w, 0.0, "bf16")
    for k in (0.25, 2.0, 64.0):
        assert orc.norm_apply((x * np.float32(k)).astype(np.float32), w, 0.0, "bf16").tobytes() == base.tobytes()
    # a missing square root is far off
    bad = orc.bf16_round((x / np.float32(np.mean(x * x))) * w)
    assert bad.tobytes() != base.tobytes()


# ---- the one-pass prefill ----------------------------------------------------

def _layer(orc, rng, dout, din, r, scale=1.0, bias=0.1):
    ubs = rng.choice([-1, 1], (dout, r)).astype(np.int8)
    vts = rng.choice([-1, 1], (r, din)).astype(np.int8)
    return dict(dout=dout, din=din, r=r, ub=orc.pack_bits(ubs), vt=orc.pack_bits(vts),
                s1=(scale * np.exp(0.3 * rng.standard_normal(dout)) / math.sqrt(r * din)).astype(np.float32),
                s2=np.exp(0.3 * rng.standard_normal(din)).astype(np.float32),
                bias=(bias * rng.standard_normal(dout)).astype(np.float32))


def _block(orc, seed, q_zero=False):
    rng = np.random.default_rng(seed)
    Ls = [_layer(orc, rng, H * HD, D, 24, 4.0), _layer(orc, rng, HK * HD, D, 24, 4.0),
          _layer(orc, rng, HK * HD, D, 24, 2.0, bias=1.0), _layer(orc, rng, D, H * HD, 24, 2.0),
          _layer(orc, rng, FFN, D, 32, 4.0), _layer(orc, rng, FFN, D, 32), _layer(orc, rng, D, FFN, 32)]
    if q_zero:
        Ls[0]["s1"] = np.zeros_like(Ls[0]["s1"])
        Ls[0]["bias"] = np.zeros_like(Ls[0]["bias"])
    norms = {"input": (1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
             "post_attention": (1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
             "q_norm": (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32),
             "k_norm": (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)}
    return Ls, norms, rng


def _dense(L):
    """A layer's dense f64 map x -> s1 * (U (Vt (s2 x))) + b from its bits."""
    def signs(rows, n, bits):
        b = np.unpackbits(bits.reshape(rows, -1), axis=1, bitorder="little")[:, :n]
        return b.astype(np.float64) * 2 - 1
    U = signs(L["dout"], L["r"], L["ub"])
    Vt = signs(L["r"], L["din"], L["vt"])
    return lambda x: L["s1"] * (U @ (Vt @ (L["s2"] * x))) + L["bias"]


def _rms(x, w):
    return x / np.sqrt((x * x).mean() + EPS) * w


def _rot(v, pos):
    v = v.reshape(-1, HD).copy()
    half = HD // 2
    ang = pos * THETA ** (-(2.0 * np.arange(half)) / HD)
    a, b = v[:, :half].copy(), v[:, half:].copy()
    v[:, :half] = a * np.cos(ang) - b * np.sin(ang)
    v[:, half:] = b * np.cos(ang) + a * np.sin(ang)
    return v.ravel()


def _dense_qkv(Ls, norms, h_rows):
    F = [_dense(L) for L in Ls]
    qs, ks, vs = [], [], []
    for t, h in enumerate(h_rows.astype(np.float64)):
        x = _rms(h, norms["input"])
        q = np.concatenate([_rms(a, norms["q_norm"]) if np.any(a) else a for a in F[0](x).reshape(H, HD)])
        k = np.concatenate([_rms(a, norms["k_norm"]) for a in F[1](x).reshape(HK, HD)])
        qs.append(_rot(q, t))
        ks.append(_rot(k, t))
        vs.append(F[2](x))
    return np.array(qs), np.array(ks), np.array(vs)


def _dense_mlp(Ls, norms, h_rows, att_rows):
    F = [_dense(L) for L in Ls]
    out = []
    for h, a in zip(h_rows.astype(np.float64), att_rows):
        h1 = F[3](a) + h
        x2 = _rms(h1, norms["post_attention"])
        g, u = F[4](x2), F[5](x2)
        out.append(F[6](g / (1 + np.exp(-g)) * u) + h1)
    return np.array(out)


def _exact_attention(q, k, v):
    """Causal softmax(q k^T / sqrt(hd)) v in f64, head h reading kv head
    h // (H / HK); rows (n, width)."""
    n = q.shape[0]
    out = np.zeros((n, H * HD))
    for h in range(H):
        kv = h // (H // HK)
        qh, kh, vh = q[:, h * HD:(h + 1) * HD], k[:, kv * HD:(kv + 1) * HD], v[:, kv * HD:(kv + 1) * HD]
        s = qh @ kh.T / math.sqrt(HD)
        s[np.triu_indices(n, 1)] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h * HD:(h + 1) * HD] = (p @ vh) / p.sum(axis=1, keepdims=True)
    return out


def _rope_late(orc, monkeypatch):
    real = orc.rope
    monkeypatch.setattr(orc, "rope", lambda v, hd, pos, th: real(v, hd, pos + 1, th))


def _no_att_rounding(orc, monkeypatch):
    monkeypatch.setattr(orc, "bf16_round", lambda x: np.asarray(x, np.float32))


def _no_transpose(orc, monkeypatch):
    def bad(rows, n_heads, head_dim):
        rows = np.asarray(rows, np.float32)
        return np.ascontiguousarray(rows.reshape(n_heads, rows.shape[0], head_dim))[None]
    monkeypatch.setattr(orc, "heads_major", bad)


N = 70    # one full 64-token key block and a ragged one


def _cache_rows_match(orc, Ls, norms, h_rows):
    kp = np.zeros((N, HK * HD), np.float32)
    vp = np.zeros_like(kp)
    orc.prefill_qkv(Ls, norms, h_rows, kp, vp, HD, THETA, EPS)
    return kp, vp


@pytest.fixture(scope="module")
def step_caches(orc):
    """The cache rows block_step (bf16 serving) writes at positions 0..N-1."""
    Ls, norms, rng = _block(orc, 11)
    h_rows = rng.standard_normal((N, D)).astype(np.float32)
    ks = np.zeros((N, HK * HD), np.float32)
    vs = np.zeros_like(ks)
    for t in range(N):
        orc.block_step(Ls, norms, h_rows[t], t, ks, vs, H, HK, HD, THETA, EPS, serving="bf16")
    return Ls, norms, h_rows, ks, vs


def test_prefill_cache_rows_equal_block_step(orc, step_caches):
    Ls, norms, h_rows, ks, vs = step_caches
    kp = np.zeros_like(ks)
    vp = np.zeros_like(vs)
    orc.block_prefill(Ls, norms, h_rows, kp, vp, H, HK, HD, THETA, EPS)
    assert kp.tobytes() == ks.tobytes()
    assert vp.tobytes() == vs.tobytes()


def test_prefill_rope_late_changes_cache_rows(orc, step_caches, monkeypatch):
    Ls, norms, h_rows, ks, vs = step_caches
    _rope_late(orc, monkeypatch)
    kp, vp = _cache_rows_match(orc, Ls, norms, h_rows)
    assert vp.tobytes() == vs.tobytes()          # v takes no RoPE
    assert np.abs(kp - ks).max() > 0.1


def _q_rows_err(orc, seed):
    Ls, norms, rng = _block(orc, seed)
    h_rows = rng.standard_normal((N, D)).astype(np.float32)
    kc = np.zeros((N, HK * HD), np.float32)
    vc = np.zeros_like(kc)
    q, k, v = orc.prefill_qkv(Ls, norms, h_rows, kc, vc, HD, THETA, EPS)
    qd, kd, vd = _dense_qkv(Ls, norms, h_rows)
    return [np.abs(a - b).max() / np.abs(b).max() for a, b in ((q, qd), (k, kd), (v, vd))]


def test_prefill_q_rows_against_dense_f64(orc, monkeypatch):
    errs = _q_rows_err(orc, 13)
    print("q/k/v rows, max rel error vs dense f64:", errs)
    assert max(errs) < 3e-2
    _rope_late(orc, monkeypatch)
    bad = _q_rows_err(orc, 13)
    print("RoPE at t + 1:", bad)
    assert bad[0] > 0.2 and bad[1] > 0.2


def _closed_form_case(seed, n=150):
    rng = np.random.default_rng(seed)
    q = np.zeros((n, H * HD), np.float32)
    k = rng.standard_normal((n, HK * HD)).astype(np.float32)
    v = rng.integers(-8, 9, (n, HK * HD)).astype(np.float32)
    want = np.zeros((n, H * HD), np.float32)
    csum = np.cumsum(v.astype(np.int64), axis=0)
    for t in range(n):
        for h in range(H):
            kv = h // (H // HK)
            s = csum[t, kv * HD:(kv + 1) * HD].astype(np.float32)
            want[t, h * HD:(h + 1) * HD] = s / np.float32(t + 1)
    return q, k, v, want


def test_prefill_attention_q0_closed_form(orc):
    """q = 0: every score is 0 (q codes 0, scale 1), p = exp2(0) = 1 for each
    visible key, so row t of head h is (sum of fp16 V over keys 0..t of kv
    head h // 2) / (t + 1): one f32 division of an exact integer sum, then
    bf16 -- bit for bit over three key blocks (the last ragged)."""
    from conftest import same

    q, k, v, want = _closed_form_case(21)
    got = orc.prefill_attention(q, k, v, H, HK, HD)
    same(got, orc.bf16_round(want), "q = 0 causal mean")


@pytest.mark.parametrize("mistake", ["no_att_rounding", "no_transpose"])
def test_prefill_attention_planted_mistakes_fail(orc, monkeypatch, mistake):
    q, k, v, want = _closed_form_case(21)
    want = orc.bf16_round(want)
    {"no_att_rounding": _no_att_rounding, "no_transpose": _no_transpose}[mistake](orc, monkeypatch)
    got = orc.prefill_attention(q, k, v, H, HK, HD)
    assert got.tobytes() != want.tobytes()


def _q0_block_err(orc, seed):
    Ls, norms, rng = _block(orc, seed, q_zero=True)
    h_rows = rng.standard_normal((N, D)).astype(np.float32)
    kc = np.zeros((N, HK * HD), np.float32)
    vc = np.zeros_like(kc)
    got = orc.block_prefill(Ls, norms, h_rows, kc, vc, H, HK, HD, THETA, EPS)
    _, _, vd = _dense_qkv(Ls, norms, h_rows)
    att = np.zeros((N, H * HD))
    mean = np.cumsum(vd, axis=0) / np.arange(1, N + 1)[:, None]
    for h in range(H):
        kv = h // (H // HK)
        att[:, h * HD:(h + 1) * HD] = mean[:, kv * HD:(kv + 1) * HD]
    want = _dense_mlp(Ls, norms, h_rows, att)
    return np.abs(got - want).max() / np.abs(want).max()


def test_block_prefill_q0_against_dense_f64(orc, monkeypatch):
    """The whole block with the q projection zeroed (s1 = bias = 0), against
    the block written densely in f64 with the attention the causal mean of V."""
    err = _q0_block_err(orc, 17)
    print("q = 0 block, max rel error vs dense f64:", err)
    assert err < 2e-2
    _no_transpose(orc, monkeypatch)
    bad = _q0_block_err(orc, 17)
    print("head-major without transpose:", bad)
    assert bad > 5e-2


def _attention_quality(orc, seed):
    Ls, norms, rng = _block(orc, seed)
    h_rows = rng.standard_normal((N, D)).astype(np.float32)
    kc = np.zeros((N, HK * HD), np.float32)
    vc = np.zeros_like(kc)
    q, k, v = orc.prefill_qkv(Ls, norms, h_rows, kc, vc, HD, THETA, EPS)
    got = orc.prefill_attention(q, k, v, H, HK, HD)
    qd, kd, vd = _dense_qkv(Ls, norms, h_rows)
    want = _exact_attention(qd, kd, vd)
    cos = min(float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b))) for a, b in zip(got, want))
    rel1 = float(np.abs(got - want).sum() / np.abs(want).sum())
    return cos, rel1


def test_prefill_attention_quality_against_exact_f64(orc, monkeypatch):
    """Real q: the attention rows against exact causal f64 attention over the
    dense block's q, k, v -- the [SA] gate (cos >= 0.999, relL1 <= 0.02)."""
    cos, rel1 = _attention_quality(orc, 19)
    print(f"attention vs exact f64: min cos {cos:.6f} relL1 {rel1:.4g}")
    assert cos >= 0.999 and rel1 <= 0.02
    # (RoPE at t + 1 on both q and k leaves every score as it is -- the
    # rotation is relative -- which is why the cache and q rows pin it.)
    _no_transpose(orc, monkeypatch)
    cos_b, rel_b = _attention_quality(orc, 19)
    print(f"head-major without transpose: min cos {cos_b:.6f} relL1 {rel_b:.4g}")
    assert cos_b < 0.999 and rel_b > 0.02
