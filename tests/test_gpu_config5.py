"""Config 5's decoder block at full size on the device (BASELINE.json
configs[4]): d 4096, 32 query / 8 KV heads of 128, FFN 14336, the config-3
ranks (q, o 1102; k, v 431; gate, up 1724; down 1733), bf16 serving; two such
blocks, the final norm and a head over an 8192-token vocabulary (the block
shapes are config 5's; the vocabulary is cut to keep the test's host memory
small).

No oracle runs at this size.  The checks are the reference's cross-face ones
(crates/quantibbler-server/tests/cross_face_sage_identity.rs,
cross_face_token_identity.rs): two device paths that compute the same
logits by different arithmetic must agree within the sage face's gate
(cosine >= 0.999 and relative L1 <= 0.02, cross_face_sage_identity.rs:84-86)
and choose the same greedy tokens.
  * prefill against decode: a 1100-token prompt through the one-pass block
    prefill (every projection on the one-launch GEMM, the causal block-scaled
    SageAttention) and through 1100 decode steps (the fp4 GEMV, the
    reference-scheme decode attention over the cache);
  * batch 32 against batch 1: one decode step of 32 sequences together (the
    projections as layer sets on the GEMM, the batched decode attention)
    against the same step of each sequence alone (the GEMV).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

D, H, HK, HD, FFN, VOCAB = 4096, 32, 8, 128, 14336, 8192
RANKS = {"q": 1102, "k": 431, "v": 431, "o": 1102, "gate": 1724, "up": 1724, "down": 1733}
CAP = 1200


def say(*a):
    print(*a, flush=True)


def _qpk1_v2(rng, dout, din, r):
    """A v2 qpk1 stream (qpk1 lib.rs:152-210): random container bitstreams
    (pad bits zero), fp16 s1 / s2 / bias."""
    s1 = (np.exp(0.3 * rng.standard_normal(dout)) / np.sqrt(r * din)).astype(np.float16)
    s2 = np.exp(0.3 * rng.standard_normal(din)).astype(np.float16)
    bias = (0.05 * rng.standard_normal(dout)).astype(np.float16)

    def bits(n):
        b = rng.integers(0, 256, (n + 7) // 8, dtype=np.uint8)
        if n % 8:
            b[-1] &= (1 << (n % 8)) - 1
        return b.tobytes()

    head = b"QPK1" + b"".join(int(v).to_bytes(4, "little") for v in (2, 1, dout, din, r))
    return head + s1.tobytes() + s2.tobytes() + bias.tobytes() + bits(dout * r) + bits(din * r)


def config5_model(seed, n_layers=2):
    from quantibbler_amd.model import ModelDir

    rng = np.random.default_rng(seed)
    streams, names = {}, []
    shapes = {"self_attn.q_proj": (H * HD, D, RANKS["q"]), "self_attn.k_proj": (HK * HD, D, RANKS["k"]),
              "self_attn.v_proj": (HK * HD, D, RANKS["v"]), "self_attn.o_proj": (D, H * HD, RANKS["o"]),
              "mlp.gate_proj": (FFN, D, RANKS["gate"]), "mlp.up_proj": (FFN, D, RANKS["up"]),
              "mlp.down_proj": (D, FFN, RANKS["down"])}
    for b in range(n_layers):
        for suffix, (m, k, r) in shapes.items():
            name = f"layers.{b}.inner.{suffix}"
            names.append(name)
            streams[name] = _qpk1_v2(rng, m, k, r)
    per_block = 2 * D + 2 * HD
    norms = (1 + 0.1 * rng.standard_normal(per_block * n_layers + D)).astype(np.float32)
    return ModelDir(path="<config 5 shape>", vocab_size=VOCAB, d_model=D, n_layers=n_layers, n_heads=H,
                    n_kv_heads=HK, head_dim=HD, rms_norm_eps=1e-5, rope_theta=500000.0,
                    norm_slots=["input", "post_attention", "q_norm", "k_norm"], remainder_dtype="f32",
                    layer_names=names, streams=streams,
                    embedding=rng.standard_normal((VOCAB, D)).astype(np.float32),
                    lm_head=(0.02 * rng.standard_normal((VOCAB, D))).astype(np.float32), norms=norms)


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


@pytest.fixture(scope="module")
def model(ctx):
    from quantibbler_amd.model import DeviceModel

    say("config 5 shape: building two blocks and the head")
    md = config5_model(555)
    m = DeviceModel(ctx, md, capacity=CAP, n_seqs=32)
    yield m
    m.close()


def sage_gate(got, want, label):
    """cosine >= 0.999 and relative L1 = sum|a - b| / sum|a| <= 0.02
    (cross_face_sage_identity.rs:84-86, 147-160); relative L2 reported."""
    g, w = np.asarray(got, np.float64), np.asarray(want, np.float64)
    cos = float(g @ w / (np.linalg.norm(g) * np.linalg.norm(w)))
    rl1 = float(np.abs(g - w).sum() / np.abs(w).sum())
    rel = float(np.linalg.norm(g - w) / np.linalg.norm(w))
    say(f"  {label}: cos {cos:.7f} relL1 {rl1:.2e} rel {rel:.2e}")
    assert np.isfinite(g).all()
    assert cos >= 0.999 and rl1 <= 0.02, (label, cos, rl1)


def test_config5_prefill_against_decode_steps(model):
    st = torch.cuda.current_stream()
    rng = np.random.default_rng(5001)
    n = 1100  # the one-launch GEMM (from 256 tokens); a ragged last group of 8
    tokens = rng.integers(0, VOCAB, n).tolist()
    say(f"config 5 shape: prefill of {n} tokens")
    model.reset()
    a = model.prefill(tokens, st).cpu().numpy().copy()
    greedy_a = []
    for _ in range(8):
        t = int(np.argmax(a if not greedy_a else la))
        greedy_a.append(t)
        la = model.step(t, st).cpu().numpy().copy()
    say(f"config 5 shape: the same {n} tokens as decode steps")
    model.reset()
    for t in tokens:
        b = model.step(t, st)
    b = b.cpu().numpy().copy()
    sage_gate(a, b, "logits after the prompt, prefill vs decode steps")
    assert int(np.argmax(a)) == int(np.argmax(b))
    greedy_b = []
    for _ in range(8):
        t = int(np.argmax(b if not greedy_b else lb))
        greedy_b.append(t)
        lb = model.step(t, st).cpu().numpy().copy()
    say(f"  greedy tokens: prefill path {greedy_a}, decode path {greedy_b}")
    assert greedy_a == greedy_b
    sage_gate(la, lb, "logits after 8 greedy steps")


def test_config5_batch32_step_matches_batch1(model):
    st = torch.cuda.current_stream()
    rng = np.random.default_rng(5002)
    lens = [int(v) for v in rng.integers(1, 70, 32)]
    prompts = [rng.integers(0, VOCAB, n).tolist() for n in lens]
    say(f"config 5 shape: 32 sequences of {min(lens)}-{max(lens)} tokens, batch 1 steps")
    model.reset()
    nxt, want, first = [], [], []
    for p in prompts:
        lg = model.prefill(p, st, seq=0).cpu().numpy().copy()
        first.append(lg)
        nxt.append(int(np.argmax(lg)))
        want.append(model.step(nxt[-1], st).cpu().numpy().copy())
    say("config 5 shape: the 32 sequences prefilled side by side, one batch-32 step")
    model.reset()
    for s, p in enumerate(prompts):
        lg = model.prefill(p, st, seq=s).cpu().numpy()
        assert np.array_equal(lg, first[s]), f"prefill of sequence {s} differs by slot"
    got = model.step_batch(nxt, st).cpu().numpy().copy()
    assert got.shape == (32, VOCAB)
    for s in range(32):
        sage_gate(got[s], want[s], f"sequence {s} ({lens[s]} tokens): batch 32 vs batch 1")
        assert int(np.argmax(got[s])) == int(np.argmax(want[s])) or \
            np.sort(want[s])[-1] - np.sort(want[s])[-2] < 1e-3 * np.abs(want[s]).max()
