"""GPU parity of the exact attention face (gpu_attention.rs:451-570
GpuContext::attention) through the C ABI:

* the reference's own battery, attention_tiled.json (9 cases: GQA, causal,
  ragged, d 4 / 128, val_dim != head_dim), against its numpy-reference
  outputs under the reference's two-part gate, rel 1e-5 with band 1e-1
  (crates/quantibbler-kernels/tests/gpu_attention_parity.rs:34-124);
* seq_q != seq_kv with the substrate's bottom-right causality (key j masked
  for query i when j + seq_q > i + seq_kv), including fully masked rows
  (NaN, as the NumPy reference gives), against a dense f64 evaluation;
* the engine's decode use (seq_q = 1 over a cache, engine/mod.rs:1041-1067)
  against the oracle's gqa_attention_scalar (engine/mod.rs:1073-1116);
* the reference's validation texts and u32 ceiling, refused before any
  device work.
"""
import math

import numpy as np
import pytest

from conftest import load_golden

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

RTOL, BAND = 1e-5, 1e-1


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def two_part(actual, expected, row_len):
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    norm = max(np.abs(a).max(), np.abs(e).max())
    assert np.isfinite(norm) and norm > 0
    assert np.abs(a - e).max() <= RTOL * norm, np.abs(a - e).max() / norm
    re, ra = e.reshape(-1, row_len), a.reshape(-1, row_len)
    rmax = np.abs(re).max(axis=1, keepdims=True)
    m = (np.abs(re) >= BAND * rmax) & (np.abs(re) > 0)
    worst = (np.abs(ra - re)[m] / np.abs(re)[m]).max() if m.any() else 0.0
    assert worst <= RTOL, worst


def test_exact_face_fixture_battery(ctx):
    from quantibbler_amd import AttentionShape

    for rec in load_golden("attention_tiled.json"):
        s = rec["shape"]
        shape = AttentionShape(s["batch"], s["n_heads"], s["n_kv_heads"], s["seq"], s["seq"], s["head_dim"],
                               s["val_dim"])
        say("exact attention", s, rec["causal"])
        q = np.array(rec["inputs"]["query"], np.float32)
        k = np.array(rec["inputs"]["key"], np.float32)
        v = np.array(rec["inputs"]["value"], np.float32)
        out = ctx.attention(shape, q, k, v, rec["causal"])
        two_part(out, np.array(rec["faces"]["numpy-reference"]["out"]), s["val_dim"])


def dense(q, k, v, causal):
    B, H, Sq, d = q.shape
    Hk, Skv = k.shape[1], k.shape[2]
    g = H // Hk
    kk, vv = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    sc = q @ kk.swapaxes(-1, -2) / math.sqrt(d)
    if causal:
        i = np.arange(Sq)[:, None]
        j = np.arange(Skv)[None, :]
        sc = np.where(j + Sq > i + Skv, -np.inf, sc)
    with np.errstate(invalid="ignore"):
        mx = sc.max(axis=-1, keepdims=True)
        p = np.exp(sc - mx)
        return (p / p.sum(axis=-1, keepdims=True)) @ vv


@pytest.mark.parametrize("sq,skv,causal", [(3, 70, True), (1, 2500, True), (5, 5, True), (40, 1100, False),
                                           (6, 4, True)])
def test_exact_face_rectangular_and_masked_rows(ctx, sq, skv, causal):
    from quantibbler_amd import AttentionShape

    say("exact attention", sq, skv, causal)
    rng = np.random.default_rng(sq * 1000 + skv)
    B, H, Hk, d, dv = 2, 4, 2, 64, 48
    q = rng.standard_normal((B, H, sq, d)).astype(np.float32)
    k = rng.standard_normal((B, Hk, skv, d)).astype(np.float32)
    v = rng.standard_normal((B, Hk, skv, dv)).astype(np.float32)
    shape = AttentionShape(B, H, Hk, sq, skv, d, dv)
    got = ctx.attention(shape, q, k, v, causal).reshape(B, H, sq, dv)
    want = dense(*(a.astype(np.float64) for a in (q, k, v)), causal)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    if (~nan).any():
        two_part(got[~nan], want[~nan], dv)
    if sq > skv and causal:
        assert nan.any()      # rows i < sq - skv see no key


def test_exact_face_decode_matches_engine_scalar(ctx, orc):
    """seq_q = 1 over a cache of pos + 1 rows: the engine's tiled decode face
    and its scalar routine solve the same problem (engine/mod.rs:1031-1116)."""
    from quantibbler_amd import AttentionShape

    rng = np.random.default_rng(77)
    H, Hk, hd, pos = 8, 2, 64, 300
    kc = rng.standard_normal((pos + 1, Hk * hd)).astype(np.float32)
    vc = rng.standard_normal((pos + 1, Hk * hd)).astype(np.float32)
    qh = rng.standard_normal(H * hd).astype(np.float32)
    want = orc.gqa_attention_scalar(qh, kc, vc, H, Hk, hd, pos)
    kh = np.ascontiguousarray(kc.reshape(pos + 1, Hk, hd).transpose(1, 0, 2))[None]
    vh = np.ascontiguousarray(vc.reshape(pos + 1, Hk, hd).transpose(1, 0, 2))[None]
    got = ctx.attention(AttentionShape(1, H, Hk, 1, pos + 1, hd, hd), qh, kh, vh, True)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    # device-pointer form: same bits as the host form
    od = torch.empty(H * hd, dtype=torch.float32, device="cuda")
    ctx.attention_dev(AttentionShape(1, H, Hk, 1, pos + 1, hd, hd), torch.from_numpy(qh).cuda(),
                      torch.from_numpy(kh).cuda(), torch.from_numpy(vh).cuda(), True, od,
                      torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert od.cpu().numpy().tobytes() == got.tobytes()


def test_exact_face_validation_texts(ctx):
    from quantibbler_amd import AttentionShape, KernelError

    q = np.zeros(8, np.float32)
    cases = [
        (AttentionShape(0, 1, 1, 1, 1, 8, 8), "attention requires non-empty batch and head dimensions"),
        (AttentionShape(1, 3, 2, 1, 1, 8, 8), "n_kv_heads must divide n_heads: n_heads=3, n_kv_heads=2"),
        (AttentionShape(1, 1, 1, 0, 1, 8, 8), "attention requires non-empty sequence and head dimensions"),
        (AttentionShape(1, 1, 1, 2, 1, 8, 8), "query must hold 16 values for AttentionShape { batch: 1, "
                                              "n_heads: 1, n_kv_heads: 1, seq_q: 2, seq_kv: 1, head_dim: 8, "
                                              "val_dim: 8 }, got 8"),
    ]
    for shape, text in cases:
        with pytest.raises(KernelError) as e:
            ctx.attention(shape, q, q, q, False)
        assert str(e.value) == text
