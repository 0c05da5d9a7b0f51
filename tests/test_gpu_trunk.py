"""GPU checks of the trunk around the decoder blocks and of the whole device
trunk on the reference's parity-tiny model:

* embedding lookup (engine/mod.rs:768-778): rows bit-identical to the table;
  the host form refuses an out-of-range id with the reference's text, the
  device form poisons that row with NaN;
* the final norm (engine/mod.rs:943, norm_apply at bf16 serving): within one
  bf16 ulp of the oracle (its sum of squares is a tree on the device);
* greedy argmax (sampler.rs:4-15): first maximum, NaN never wins, 0 when
  nothing beats -inf -- bit-exact on the edge cases;
* DeviceModel (embedding -> 2 blocks with q/k norms -> final norm -> lm_head
  on the device, bf16 serving, sage decode attention) on
  tests/fixtures/parity-tiny: every position's logits within the reference's
  1e-2 budget of the HF goldens (crates/quantibbler-server/tests/
  parity_tiny.rs:25-100), and close to the oracle's trunk in the same
  configuration.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TINY = os.path.join(GOLDEN, "parity_tiny")


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def test_embed_host_and_device(ctx):
    from quantibbler_amd import KernelError
    from quantibbler_amd.gpu import embed, embed_dev

    say("trunk embed")
    rng = np.random.default_rng(5)
    vocab, d = 300, 96
    table = rng.standard_normal((vocab, d)).astype(np.float32)
    td = torch.from_numpy(table).cuda()
    ids = np.array([0, 299, 17, 17, 5], np.int32)
    out = torch.empty((5, d), dtype=torch.float32, device="cuda")
    embed(ctx, td, vocab, d, ids, out)
    assert np.array_equal(out.cpu().numpy(), table[ids])
    with pytest.raises(KernelError, match=r"token id 300 is outside the vocabulary \(size 300\)"):
        embed(ctx, td, vocab, d, np.array([1, 300], np.int32), out)
    idd = torch.tensor([3, -1, 400, 299], dtype=torch.int32, device="cuda")
    out4 = torch.empty((4, d), dtype=torch.float32, device="cuda")
    embed_dev(ctx, td, vocab, d, idd, 4, out4, torch.cuda.current_stream())
    torch.cuda.synchronize()
    o = out4.cpu().numpy()
    assert np.array_equal(o[0], table[3]) and np.array_equal(o[3], table[299])
    assert np.isnan(o[1]).all() and np.isnan(o[2]).all()


def test_final_norm_against_oracle(ctx, orc):
    from quantibbler_amd.gpu import rms_norm_dev

    say("trunk final norm")
    rng = np.random.default_rng(6)
    for d in (64, 4096, 4099):
        x = (3 * rng.standard_normal((3, d))).astype(np.float32)
        w = orc.bf16_to_f32(orc.f32_to_bf16((1 + 0.1 * rng.standard_normal(d)).astype(np.float32)))
        xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
        od = torch.empty_like(xd)
        rms_norm_dev(ctx, xd, 3, d, wd, 1e-5, od, torch.cuda.current_stream())
        torch.cuda.synchronize()
        got = od.cpu().numpy()
        for r in range(3):
            want = orc.norm_apply(x[r], w, 1e-5, "bf16")
            assert np.array_equal(orc.bf16_to_f32(orc.f32_to_bf16(got[r])), got[r])   # bf16 values
            ulp = np.spacing(np.abs(want).astype(np.float32)) * 2 ** 16
            assert np.all(np.abs(got[r] - want) <= ulp), (d, r)


def greedy(row):
    best, best_v = 0, -np.inf
    for i, v in enumerate(row):
        if v > best_v:
            best, best_v = i, v
    return best


def test_argmax_first_max_rule(ctx):
    from quantibbler_amd.gpu import argmax_dev

    say("trunk argmax")
    rng = np.random.default_rng(7)
    vocab = 1000
    rows = [rng.standard_normal(vocab).astype(np.float32) for _ in range(4)]
    r = rng.integers(-3, 3, vocab).astype(np.float32)          # many ties at the max
    rows.append(r)
    r = np.full(vocab, -np.inf, np.float32)                      # nothing beats -inf
    rows.append(r)
    r = np.full(vocab, np.nan, np.float32)
    r[[10, 900]] = 2.0                                            # NaN never wins; first of ties
    rows.append(r)
    r = rng.standard_normal(vocab).astype(np.float32)
    r[0] = np.nan
    r[999] = 50.0
    rows.append(r)
    x = np.stack(rows)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty(len(rows), dtype=torch.int32, device="cuda")
    argmax_dev(ctx, xd, len(rows), vocab, out, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert out.cpu().numpy().tolist() == [greedy(row) for row in rows]


@pytest.mark.parametrize("vocab", [1, 3, 7, 128256, 128259])
def test_argmax_wide_rows(ctx, vocab):
    """Rows of odd length start off the 16-byte grid (the kernel's scalar
    head), long rows take the vector body and a scalar tail; the winner is
    placed in each part, with ties between the parts."""
    from quantibbler_amd.gpu import argmax_dev

    say(f"trunk argmax wide rows vocab={vocab}")
    rng = np.random.default_rng(vocab)
    rows = []
    for pos in sorted({0, 1, 2, vocab // 2, vocab - 2, vocab - 1}):
        if not 0 <= pos < vocab:
            continue
        r = rng.standard_normal(vocab).astype(np.float32)
        r[pos] = 9.0
        rows.append(r)
        t = r.copy()
        t[vocab - 1 - pos] = 9.0                                  # a tie: the first index wins
        rows.append(t)
    r = np.full(vocab, np.nan, np.float32)
    r[-1] = -1.0
    rows.append(r)
    x = np.stack(rows)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty(len(rows), dtype=torch.int32, device="cuda")
    argmax_dev(ctx, xd, len(rows), vocab, out, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert out.cpu().numpy().tolist() == [int(np.argmax(np.nan_to_num(row, nan=-np.inf))) for row in rows]


@pytest.fixture(scope="module")
def md():
    from quantibbler_amd.model import ModelDir

    return ModelDir.load(TINY)


def test_device_trunk_parity_tiny_goldens(ctx, orc, md):
    from quantibbler_amd.model import DeviceModel

    say("device trunk on parity-tiny")
    with open(os.path.join(TINY, "goldens.json")) as f:
        g = json.load(f)
    ids = g["input_ids"]
    m = DeviceModel(ctx, md, capacity=16)
    ref = orc.Trunk(md, serving="bf16", attention="sage", capacity=16)
    worst_gold, worst_orc = 0.0, 0.0
    for pos, tok in enumerate(ids):
        logits = m.step(tok, torch.cuda.current_stream())
        torch.cuda.synchronize()
        got = logits.cpu().numpy()
        want = ref.step(tok)
        gold = np.array(g["logits"][pos], np.float32)
        worst_gold = max(worst_gold, float(np.abs(got - gold).max()))
        worst_orc = max(worst_orc, float(np.abs(got - want).max()))
        say(f"  pos {pos}: |device - HF| {np.abs(got - gold).max():.3g}  |device - oracle| "
            f"{np.abs(got - want).max():.3g}")
    assert worst_gold <= 1e-2, worst_gold
    assert worst_orc <= 2e-3, worst_orc
    # a fresh sequence after reset reproduces the first position
    m.reset()
    again = m.step(ids[0], torch.cuda.current_stream()).cpu().numpy()
    ref0 = orc.Trunk(md, serving="bf16", attention="sage", capacity=16).step(ids[0])
    assert np.abs(again - ref0).max() <= 2e-3
    m.close()


def test_device_trunk_exact_face(ctx, orc, md):
    """The trunk on the exact attention face (DeviceModel(attention="exact"):
    every block's engine/mod.rs:1041-1067 face) against the oracle on the
    reference's default scalar face and the HF goldens; then the reference's
    cross-face scenario (crates/quantibbler-server/tests/
    cross_face_sage_identity.rs): greedy generation through the exact face and
    through the sage face from the same prompt yields the same tokens, and the
    final logits agree within the sage face's gate."""
    from quantibbler_amd.model import DeviceModel

    say("device trunk on parity-tiny, exact face")
    with open(os.path.join(TINY, "goldens.json")) as f:
        g = json.load(f)
    ids = g["input_ids"]
    cap = len(ids) + 8
    m = DeviceModel(ctx, md, capacity=cap, attention="exact")
    ref = orc.Trunk(md, serving="bf16", attention="scalar", capacity=cap)
    worst_gold, worst_orc = 0.0, 0.0
    st = torch.cuda.current_stream()
    for pos, tok in enumerate(ids):
        got = m.step(tok, st).cpu().numpy()
        want = ref.step(tok)
        gold = np.array(g["logits"][pos], np.float32)
        worst_gold = max(worst_gold, float(np.abs(got - gold).max()))
        rel_inf = float(np.abs(got - want).max() / np.abs(want).max())
        worst_orc = max(worst_orc, rel_inf)
        say(f"  pos {pos}: |device - HF| {np.abs(got - gold).max():.3g}  |device - oracle (scalar face)| "
            f"{np.abs(got - want).max():.3g} (rel inf-norm {rel_inf:.3g})")
    assert worst_gold <= 1e-2, worst_gold
    # the exact faces' reassociation budget (cross_face_token_identity.rs:
    # rel inf-norm <= 1e-5); measured 0 here
    assert worst_orc <= 1e-5, worst_orc
    # cross-face: the same prompt, then greedy steps, on each face
    streams = {}
    for face in ("exact", "sage"):
        mf = m if face == "exact" else DeviceModel(ctx, md, capacity=cap, attention="sage")
        mf.reset()
        for t in ids[:4]:  # forward_prefill's per-token loop (engine/mod.rs:811-822)
            logits = mf.step(t, st)
        logits = logits.cpu().numpy().copy()
        toks = []
        for _ in range(6):
            t = greedy(logits)
            toks.append(t)
            logits = mf.step(t, st).cpu().numpy().copy()
        streams[face] = (toks, logits)
        if mf is not m:
            mf.close()
    say(f"  greedy tokens: exact {streams['exact'][0]}, sage {streams['sage'][0]}")
    assert streams["exact"][0] == streams["sage"][0]
    sage_gate(streams["sage"][1], streams["exact"][1], "final logits, sage face vs exact face")
    m.close()


@pytest.mark.parametrize("face", ["exact", "sage"])
def test_device_trunk_fp32_serving(ctx, orc, md, face):
    """The trunk at fp32 serving (engine/mod.rs ServingDtype::Fp32: apply's
    f64 products, f32 norms, the remainder tensors as stored) on each
    attention face, against the oracle's fp32 trunk on the same face within
    the exact faces' budget (relative inf-norm <= 1e-5,
    cross_face_token_identity.rs) and the HF goldens of parity-tiny (the
    oracle reproduces them to 8.6e-5 at fp32 serving)."""
    from quantibbler_amd.model import DeviceModel

    say(f"device trunk on parity-tiny, fp32 serving, {face} face")
    with open(os.path.join(TINY, "goldens.json")) as f:
        g = json.load(f)
    ids = g["input_ids"]
    cap = len(ids) + 4
    m = DeviceModel(ctx, md, capacity=cap, attention=face, serving="fp32")
    ref = orc.Trunk(md, serving="fp32", attention="scalar" if face == "exact" else "sage", capacity=cap)
    worst_gold, worst_orc = 0.0, 0.0
    st = torch.cuda.current_stream()
    for pos, tok in enumerate(ids):
        got = m.step(tok, st).cpu().numpy()
        want = ref.step(tok)
        gold = np.array(g["logits"][pos], np.float32)
        rel_inf = float(np.abs(got - want).max() / np.abs(want).max())
        worst_gold = max(worst_gold, float(np.abs(got - gold).max()))
        worst_orc = max(worst_orc, rel_inf)
        say(f"  pos {pos}: |device - HF| {np.abs(got - gold).max():.3g}  rel inf-norm to the oracle {rel_inf:.3g}")
    assert worst_orc <= 1e-5, worst_orc
    assert worst_gold <= (1e-3 if face == "exact" else 1e-2), worst_gold
    m.close()


def _qpk1_v2(orc, rng, dout, din, r):
    """A random v2 qpk1 layer stream (f16 scales and bias), as the reference's
    writer lays it out (container bitstreams, element (i, j) at bit i r + j)."""
    ubs = rng.choice([0, 1], (dout, r)).astype(np.uint8)
    vbs = rng.choice([0, 1], (din, r)).astype(np.uint8)
    s1 = (np.exp(0.3 * rng.standard_normal(dout)) / np.sqrt(r * din)).astype(np.float16)
    s2 = np.exp(0.3 * rng.standard_normal(din)).astype(np.float16)
    bias = (0.05 * rng.standard_normal(dout)).astype(np.float16)
    head = b"QPK1" + b"".join(int(v).to_bytes(4, "little") for v in (2, 1, dout, din, r))
    return (head + s1.tobytes() + s2.tobytes() + bias.tobytes()
            + np.packbits(ubs.ravel(), bitorder="little").tobytes()
            + np.packbits(vbs.ravel(), bitorder="little").tobytes())


def synthetic_model(orc, seed, vocab=300, d=256, n_layers=2, H=4, Hk=2, hd=128, ffn=512):
    from quantibbler_amd.model import ModelDir

    rng = np.random.default_rng(seed)
    streams, names = {}, []
    for b in range(n_layers):
        for suffix, (m, k, r) in (("self_attn.q_proj", (H * hd, d, 48)), ("self_attn.k_proj", (Hk * hd, d, 32)),
                                  ("self_attn.v_proj", (Hk * hd, d, 32)), ("self_attn.o_proj", (d, H * hd, 48)),
                                  ("mlp.gate_proj", (ffn, d, 64)), ("mlp.up_proj", (ffn, d, 64)),
                                  ("mlp.down_proj", (d, ffn, 64))):
            name = f"layers.{b}.inner.{suffix}"
            names.append(name)
            streams[name] = _qpk1_v2(orc, rng, m, k, r)
    per_block = 2 * d + 2 * hd
    norms = (1 + 0.1 * rng.standard_normal(per_block * n_layers + d)).astype(np.float32)
    return ModelDir(path="<synthetic>", vocab_size=vocab, d_model=d, n_layers=n_layers, n_heads=H, n_kv_heads=Hk,
                    head_dim=hd, rms_norm_eps=1e-6, rope_theta=10000.0,
                    norm_slots=["input", "post_attention", "q_norm", "k_norm"], remainder_dtype="f32",
                    layer_names=names, streams=streams,
                    embedding=rng.standard_normal((vocab, d)).astype(np.float32),
                    lm_head=(0.1 * rng.standard_normal((vocab, d))).astype(np.float32), norms=norms)


def test_device_trunk_prefill_then_decode(ctx, orc):
    """DeviceModel.prefill (every block's one-pass prefill: batched
    projections, causal block-scaled SageAttention) and then greedy decode
    steps, against the oracle composing the same arithmetic block by block
    (block_prefill, then block_step on the caches it filled)."""
    from quantibbler_amd.model import DeviceModel, _bf16_values

    say("device trunk prefill + decode")
    md = synthetic_model(orc, 808)
    n = 70
    rng = np.random.default_rng(809)
    tokens = rng.integers(0, md.vocab_size, n).tolist()
    m = DeviceModel(ctx, md, capacity=128)
    got = m.prefill(tokens, torch.cuda.current_stream()).cpu().numpy()
    # oracle: the same per-block arithmetic
    ref = orc.Trunk(md, serving="bf16", attention="sage", capacity=128)
    h = ref.embedding[np.array(tokens)].copy()
    for b, (layers, norms) in enumerate(ref.blocks):
        h = orc.block_prefill(layers, norms, h, ref.kc[b], ref.vc[b], md.n_heads, md.n_kv_heads, md.head_dim,
                              md.rope_theta, md.rms_norm_eps)
    ref.pos = n
    hn = orc.norm_apply(h[-1], ref.final_norm, md.rms_norm_eps, "bf16")
    want = orc.head_logits(ref.head, hn)
    sage_gate(got, want, "prefill")
    assert int(np.argmax(got)) == int(np.argmax(want)) or np.sort(want)[-1] - np.sort(want)[-2] < 1e-2
    for _ in range(3):
        tok = int(np.argmax(want))
        got = m.step(tok, torch.cuda.current_stream()).cpu().numpy()
        want = ref.step(tok)
        sage_gate(got, want, "decode")
    m.close()


def sage_gate(got, want, label):
    """The reference's gate for final logits on the sage face
    (crates/quantibbler-server/tests/cross_face_sage_identity.rs:84-86,
    147-160): cosine >= 0.999 and relative L1 = sum|a - b| / sum|a| <= 0.02;
    the relative L2 is reported beside them."""
    g, w = np.asarray(got, np.float64), np.asarray(want, np.float64)
    cos = float(g @ w / (np.linalg.norm(g) * np.linalg.norm(w)))
    rl1 = float(np.abs(g - w).sum() / np.abs(w).sum())
    rel = float(np.linalg.norm(g - w) / np.linalg.norm(w))
    say(f"  {label} logits cos {cos:.7f} relL1 {rl1:.2e} rel {rel:.2e}")
    assert cos >= 0.999 and rl1 <= 0.02, (label, cos, rl1)


def _oracle_prefill(orc, md, tokens, capacity):
    """The oracle trunk of one sequence after its prefill: the per-block
    arithmetic DeviceModel.prefill runs (block_prefill over the tokens'
    embedding rows), and the last position's logits."""
    ref = orc.Trunk(md, serving="bf16", attention="sage", capacity=capacity)
    h = ref.embedding[np.array(tokens)].copy()
    for b, (layers, norms) in enumerate(ref.blocks):
        h = orc.block_prefill(layers, norms, h, ref.kc[b], ref.vc[b], md.n_heads, md.n_kv_heads, md.head_dim,
                              md.rope_theta, md.rms_norm_eps)
    ref.pos = len(tokens)
    hn = orc.norm_apply(h[-1], ref.final_norm, md.rms_norm_eps, "bf16")
    return ref, orc.head_logits(ref.head, hn)


def test_device_trunk_batched_greedy(ctx, orc):
    """Batched serving: ten sequences, each prefilled to its own length, then
    greedy steps of all ten together (DeviceModel.step_batch: projections at
    batch 10 on the GEMM, every sequence's attention on its own cache), the
    ids once from the host and once as a device tensor, then a step of the
    first three (batch 3, the GEMV): each sequence's logits against its own
    oracle trunk, which takes the same greedy ids.

    Every row is held to the reference's sage-face gate on final logits
    (cosine >= 0.999, relative L1 <= 0.02: cross_face_sage_identity.rs:84-86),
    as the single-sequence trunk test holds its rows; the relative L2 of each
    row is reported beside it."""
    from quantibbler_amd.model import DeviceModel

    say("device trunk batched greedy decode")
    md = synthetic_model(orc, 818)
    lens = [70, 3, 1, 20, 64, 65, 9, 2, 33, 5]
    ns, cap = len(lens), 96
    rng = np.random.default_rng(819)
    m = DeviceModel(ctx, md, capacity=cap, n_seqs=ns)
    st = torch.cuda.current_stream()
    refs, nxt, rels = [], [], []
    for s, n in enumerate(lens):
        tokens = rng.integers(0, md.vocab_size, n).tolist()
        got = m.prefill(tokens, st, seq=s).cpu().numpy()
        ref, want = _oracle_prefill(orc, md, tokens, cap)
        sage_gate(got, want, f"prefill of sequence {s}")
        rels.append(float(np.linalg.norm(got - want) / np.linalg.norm(want)))
        refs.append(ref)
        nxt.append(int(np.argmax(want)))
    say(f"  prefill logits rel per sequence: {' '.join(f'{r:.1e}' for r in rels)}")
    assert m.positions == lens
    for step, n in enumerate((ns, ns, 3)):
        ids = nxt[:n] if step != 1 else torch.tensor(nxt[:n], dtype=torch.int32, device="cuda")
        got = m.step_batch(ids, st).cpu().numpy()
        assert got.shape == (n, md.vocab_size)
        row = []
        for s in range(n):
            want = refs[s].step(nxt[s])
            sage_gate(got[s], want, f"batch {n} step, sequence {s}")
            row.append(float(np.linalg.norm(got[s] - want) / np.linalg.norm(want)))
            nxt[s] = int(np.argmax(want))
        say(f"  batch {n}: logits rel per sequence: {' '.join(f'{r:.1e}' for r in row)}")
        rels += row
    say(f"  relative L2: mean {np.mean(rels):.2e}, max {np.max(rels):.2e} over {len(rels)} rows")
    assert m.positions == [p + 3 for p in lens[:3]] + [p + 2 for p in lens[3:]]
    with pytest.raises(ValueError, match="a batch of 11 sequences on a model holding 10"):
        m.step_batch([0] * 11, st)
    m.close()
