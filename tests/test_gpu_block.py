"""GPU check: one decoder block at one position (engine/mod.rs:878-945, bf16
serving, sage decode attention) through the C ABI, against the oracle's
restatement over a run of positions that crosses key-block boundaries.

The block's projections are the device factor linears, whose f32 sums run in
MFMA order (the reference sums each row sequentially), its norms' sums are
trees and its exp is the device's, so the block is held to a tolerance: per
position, cosine and relative L2 error of the output against the oracle fed
the same inputs (each position a fresh input, as a new token's embedding
would be; the caches of the two sides grow separately)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

COS_MIN = 0.9999
REL_MAX = 0.01
# fp32 serving (f64 products): the block's tree-summed norms and device exps
# against the reference's sequential sums and libm exps
F32_COS_MIN = 0.9999999
F32_REL_MAX = 1e-5  # the exact faces' budget (cross_face_token_identity.rs: rel <= 1e-5)


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def scaled_layer(orc, rng, dout, din, r):
    """Random signs; scales that keep |y| near |x| (s1 ~ 1/sqrt(r din))."""
    ubs = rng.choice([-1, 1], (dout, r)).astype(np.int8)
    vts = rng.choice([-1, 1], (r, din)).astype(np.int8)
    s2 = np.exp(0.3 * rng.standard_normal(din)).astype(np.float32)
    s1 = (np.exp(0.3 * rng.standard_normal(dout)) / np.sqrt(r * din)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(dout)).astype(np.float32)
    return dict(dout=dout, din=din, r=r, ub=orc.pack_bits(ubs), vt=orc.pack_bits(vts), s1=s1, s2=s2,
                bias=bias)


def metrics(got, want):
    got, want = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    cos = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want) + 1e-300))
    rel = float(np.linalg.norm(got - want) / (np.linalg.norm(want) + 1e-300))
    return cos, rel


@pytest.mark.parametrize("qk_norm", [False, True])
def test_decoder_block_matches_oracle(ctx, orc, qk_norm):
    from quantibbler_amd import DecoderBlock, FactorLayer

    d, H, Hk, hd, ffn, cap, blk = 256, 4, 2, 64, 512, 40, 16
    theta, eps = 500000.0, 1e-5
    rng = np.random.default_rng(17 + qk_norm)
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    bfv = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    norms = {"input": bfv(1.0 + 0.1 * rng.standard_normal(d)), "post_attention": bfv(1.0 + 0.1 * rng.standard_normal(d))}
    if qk_norm:
        norms["q_norm"] = bfv(1.0 + 0.2 * rng.standard_normal(hd))
        norms["k_norm"] = bfv(1.0 + 0.2 * rng.standard_normal(hd))
    block = DecoderBlock(ctx, devs, norms["input"], norms["post_attention"], H, Hk, hd, theta, eps, cap, blk,
                         norms.get("q_norm"), norms.get("k_norm"))
    kc = np.zeros((cap, Hk * hd), np.float32)
    vc = np.zeros((cap, Hk * hd), np.float32)
    assert all(block.cache_ptrs())
    st = torch.cuda.current_stream()
    worst = (1.0, 0.0)
    for pos in range(20):
        h = rng.standard_normal(d).astype(np.float32)
        hd_dev = torch.from_numpy(h).cuda()
        block.decode_dev(hd_dev, pos, st)
        torch.cuda.synchronize()
        want = orc.block_step(layers, norms, h, pos, kc, vc, H, Hk, hd, theta, eps, "bf16", "sage", blk)
        got = hd_dev.cpu().numpy()
        cos, rel = metrics(got, want)
        print(f"pos {pos}: out cos {cos:.7f} rel {rel:.2e}", flush=True)
        worst = (min(worst[0], cos), max(worst[1], rel))
        assert cos >= COS_MIN and rel <= REL_MAX, (pos, cos, rel)
    print("worst", worst, flush=True)
    block.close()


def _small_block(ctx, orc, seed, qk_norm, cap=40, blk=16):
    from quantibbler_amd import DecoderBlock, FactorLayer

    d, H, Hk, hd, ffn = 256, 4, 2, 64, 512
    rng = np.random.default_rng(seed)
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    bfv = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    norms = {"input": bfv(1.0 + 0.1 * rng.standard_normal(d)),
             "post_attention": bfv(1.0 + 0.1 * rng.standard_normal(d))}
    if qk_norm:
        norms["q_norm"] = bfv(1.0 + 0.2 * rng.standard_normal(hd))
        norms["k_norm"] = bfv(1.0 + 0.2 * rng.standard_normal(hd))
    block = DecoderBlock(ctx, devs, norms["input"], norms["post_attention"], H, Hk, hd, 500000.0, 1e-5, cap, blk,
                         norms.get("q_norm"), norms.get("k_norm"))
    return block, layers, norms, rng, dict(d=d, H=H, Hk=Hk, hd=hd, cap=cap, blk=blk)


@pytest.mark.parametrize("qk_norm", [False, True])
def test_decoder_block_exact_face_matches_oracle(ctx, orc, qk_norm):
    """The exact attention face (engine/mod.rs:1041-1067, the f32 attention the
    scalar default face also computes, :1073-1116) against the oracle's block
    step on the scalar face; positions 8-15 switch the block to the sage face
    and back (the oracle's sage face recomputes from the cache each step, so
    the device's kept state must rebuild the rows the exact face wrote)."""
    block, layers, norms, rng, g = _small_block(ctx, orc, 31 + qk_norm, qk_norm)
    kc = np.zeros((g["cap"], g["Hk"] * g["hd"]), np.float32)
    vc = np.zeros((g["cap"], g["Hk"] * g["hd"]), np.float32)
    st = torch.cuda.current_stream()
    worst = {"exact": (1.0, 0.0), "sage": (1.0, 0.0)}
    for pos in range(24):
        face = "sage" if 8 <= pos < 16 else "exact"
        block.set_attention_face(face)
        h = rng.standard_normal(g["d"]).astype(np.float32)
        hd_dev = torch.from_numpy(h).cuda()
        block.decode_dev(hd_dev, pos, st)
        torch.cuda.synchronize()
        want = orc.block_step(layers, norms, h, pos, kc, vc, g["H"], g["Hk"], g["hd"], 500000.0, 1e-5, "bf16",
                              "scalar" if face == "exact" else "sage", g["blk"])
        cos, rel = metrics(hd_dev.cpu().numpy(), want)
        say(f"pos {pos} ({face}): out cos {cos:.8f} rel {rel:.2e}")
        w = worst[face]
        worst[face] = (min(w[0], cos), max(w[1], rel))
        assert cos >= COS_MIN and rel <= REL_MAX, (pos, face, cos, rel)
    say("worst", worst)
    block.close()


def test_decoder_block_exact_face_prefill_and_refusals(ctx, orc):
    """On the exact face the prefill is forward_prefill's per-token loop
    (engine/mod.rs:811-822): bit-identical to the same rows as decode steps;
    the batched and device-position steps refuse the face."""
    from quantibbler_amd import KernelError

    block, layers, norms, rng, g = _small_block(ctx, orc, 41, True)
    block.set_attention_face("exact")
    st = torch.cuda.current_stream()
    n = 21
    rows = rng.standard_normal((n, g["d"])).astype(np.float32)
    a = torch.from_numpy(rows).cuda()
    need = block.prefill_workspace_size(n)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    block.prefill_dev(a, n, ws, need, st)
    block.reset()
    b = torch.from_numpy(rows).cuda()
    for t in range(n):
        block.decode_dev(b[t], t, st)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    h = torch.zeros(g["d"], dtype=torch.float32, device="cuda")
    nb = block.decode_batch_workspace_size(1)
    wsb = torch.empty(nb, dtype=torch.uint8, device="cuda")
    with pytest.raises(KernelError, match="the exact attention face serves one sequence at host positions"):
        block.decode_batch_dev(h, [n], wsb, nb, st)
    pos = torch.tensor([n], dtype=torch.int32, device="cuda")
    with pytest.raises(KernelError, match="the exact attention face serves one sequence at host positions"):
        block.decode_pos_dev(h, pos, st)
    with pytest.raises(KernelError, match=r"attention face must be one of \['exact', 'sage'\], got 'tiled'"):
        block.set_attention_face("tiled")
    block.close()


@pytest.mark.parametrize("face", ["exact", "sage"])
def test_decoder_block_fp32_serving_matches_oracle(ctx, orc, face):
    """fp32 serving (engine/mod.rs ServingDtype::Fp32: apply's f64 products,
    f32 norms) on each attention face, against the oracle's block step at
    fp32 serving.  The products are the reference's f64 row sums; the norms'
    sums are trees and the exps the device's, hence a tolerance, far tighter
    than bf16 serving's."""
    block, layers, norms, rng, g = _small_block(ctx, orc, 51 + (face == "sage"), True)
    block.set_serving("fp32")
    block.set_attention_face(face)
    kc = np.zeros((g["cap"], g["Hk"] * g["hd"]), np.float32)
    vc = np.zeros((g["cap"], g["Hk"] * g["hd"]), np.float32)
    st = torch.cuda.current_stream()
    worst = (1.0, 0.0)
    for pos in range(20):
        h = rng.standard_normal(g["d"]).astype(np.float32)
        hd_dev = torch.from_numpy(h).cuda()
        block.decode_dev(hd_dev, pos, st)
        torch.cuda.synchronize()
        want = orc.block_step(layers, norms, h, pos, kc, vc, g["H"], g["Hk"], g["hd"], 500000.0, 1e-5, "fp32",
                              "scalar" if face == "exact" else "sage", g["blk"])
        cos, rel = metrics(hd_dev.cpu().numpy(), want)
        say(f"fp32 pos {pos} ({face}): out cos {cos:.9f} rel {rel:.2e}")
        worst = (min(worst[0], cos), max(worst[1], rel))
        assert cos >= F32_COS_MIN and rel <= F32_REL_MAX, (pos, face, cos, rel)
    say("fp32 worst", face, worst)
    # the token-by-token prefill equals the same rows as decode steps; the
    # batched step refuses fp32 serving
    from quantibbler_amd import KernelError

    n = 9
    rows = rng.standard_normal((n, g["d"])).astype(np.float32)
    a = torch.from_numpy(rows).cuda()
    need = block.prefill_workspace_size(n)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    block.reset()
    block.prefill_dev(a, n, ws, need, st)
    block.reset()
    b = torch.from_numpy(rows).cuda()
    for t in range(n):
        block.decode_dev(b[t], t, st)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    nb = block.decode_batch_workspace_size(1)
    wsb = torch.empty(nb, dtype=torch.uint8, device="cuda")
    if face == "sage":
        with pytest.raises(KernelError, match="fp32 serving runs one sequence at host positions"):
            block.decode_batch_dev(b[0], [n], wsb, nb, st)
    block.close()


def test_decoder_block_validation(ctx, orc):
    from quantibbler_amd import DecoderBlock, FactorLayer, KernelError

    rng = np.random.default_rng(23)
    d, H, Hk, hd, ffn = 128, 2, 1, 64, 256
    shapes = [(H * hd, d, 16), (Hk * hd, d, 16), (Hk * hd, d, 16), (d, H * hd, 16),
              (ffn, d, 16), (ffn, d, 16), (d, ffn, 16)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    w = np.ones(d, np.float32)
    with pytest.raises(KernelError, match=r"decoder block: k is 128x128, expected 64x128"):
        DecoderBlock(ctx, [devs[0], devs[0]] + devs[2:], w, w, H, Hk, hd, 1e4, 1e-5, 16)
    with pytest.raises(KernelError, match="n_kv_heads dividing n_heads"):
        DecoderBlock(ctx, devs, w, w, 3, 2, hd, 1e4, 1e-5, 16)
    with pytest.raises(KernelError, match="norm weights of 127 and 128 floats; d_model is 128"):
        DecoderBlock(ctx, devs, w[:127], w, H, Hk, hd, 1e4, 1e-5, 16)
    with pytest.raises(KernelError, match="q/k norm weights of 32 floats; head_dim is 64"):
        DecoderBlock(ctx, devs, w, w, H, Hk, hd, 1e4, 1e-5, 16, 16, w[:32], w[:32])
    with pytest.raises(KernelError, match="q_norm and k_norm come together"):
        DecoderBlock(ctx, devs, w, w, H, Hk, hd, 1e4, 1e-5, 16, 16, w[:64], None)
    block = DecoderBlock(ctx, devs, w, w, H, Hk, hd, 1e4, 1e-5, 4, 16)
    h = torch.zeros(d, dtype=torch.float32, device="cuda")
    with pytest.raises(KernelError, match="position 4 is past the block's cache capacity of 4"):
        block.decode_dev(h, 4)
    with pytest.raises(KernelError, match="position 2 skips cache rows: the block holds 0 positions"):
        block.decode_dev(h, 2)
    for bad in (torch.zeros(d, dtype=torch.float32), torch.zeros(d, dtype=torch.bfloat16, device="cuda"),
                torch.zeros(d - 1, dtype=torch.float32, device="cuda"),
                torch.zeros(2 * d, dtype=torch.float32, device="cuda")[::2]):
        with pytest.raises(KernelError, match="contiguous float32 device tensor of 128 values"):
            block.decode_dev(bad, 0)
    block.decode_dev(h, 0)
    block.decode_dev(h, 1)
    block.decode_dev(h, 1)      # a rewind to position 1 is allowed
    torch.cuda.synchronize()
    assert bool(torch.isfinite(h).all())
    block.close()


@pytest.mark.parametrize("n", [5, 150])
def test_block_prefill_then_decode(ctx, orc, n):
    """A new sequence's n tokens in one prefill pass (projections at batch n:
    the decode GEMV for n <= 32, the GEMM beyond; causal block-scaled
    SageAttention over the n tokens; q/k norms; cache rows 0 .. n - 1), then
    decode steps at positions n, n + 1, ... on the cache it filled: each row
    against the oracle's restatement of the same arithmetic, to the block's
    tolerance."""
    from quantibbler_amd import DecoderBlock, FactorLayer

    d, H, Hk, hd, ffn, cap, blk = 256, 4, 2, 128, 512, 200, 64
    theta, eps = 500000.0, 1e-5
    rng = np.random.default_rng(300 + n)
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    bfv = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    norms = {"input": bfv(1.0 + 0.1 * rng.standard_normal(d)), "post_attention": bfv(1.0 + 0.1 * rng.standard_normal(d)),
             "q_norm": bfv(1.0 + 0.2 * rng.standard_normal(hd)), "k_norm": bfv(1.0 + 0.2 * rng.standard_normal(hd))}
    block = DecoderBlock(ctx, devs, norms["input"], norms["post_attention"], H, Hk, hd, theta, eps, cap, blk,
                         norms["q_norm"], norms["k_norm"])
    h = rng.standard_normal((n, d)).astype(np.float32)
    hdv = torch.from_numpy(h).cuda()
    wn = block.prefill_workspace_size(n)
    ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    block.prefill_dev(hdv, n, ws, wn, st)
    torch.cuda.synchronize()
    kc = np.zeros((cap, Hk * hd), np.float32)
    vc = np.zeros((cap, Hk * hd), np.float32)
    want = orc.block_prefill(layers, norms, h, kc, vc, H, Hk, hd, theta, eps)
    got = hdv.cpu().numpy()
    worst = (1.0, 0.0)
    for t in range(n):
        cos, rel = metrics(got[t], want[t])
        worst = (min(worst[0], cos), max(worst[1], rel))
    print(f"prefill n={n}: worst cos {worst[0]:.7f} rel {worst[1]:.2e}", flush=True)
    assert worst[0] >= COS_MIN and worst[1] <= REL_MAX, worst
    for pos in range(n, n + 4):
        x = rng.standard_normal(d).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        block.decode_dev(xd, pos, st)
        torch.cuda.synchronize()
        w2 = orc.block_step(layers, norms, x, pos, kc, vc, H, Hk, hd, theta, eps, "bf16", "sage", blk)
        cos, rel = metrics(xd.cpu().numpy(), w2)
        print(f"decode after prefill, pos {pos}: cos {cos:.7f} rel {rel:.2e}", flush=True)
        assert cos >= COS_MIN and rel <= REL_MAX, (pos, cos, rel)
    block.close()


def test_block_batched_decode(ctx, orc):
    """A block holding ten sequences: each prefilled to its own length (0 ..
    130 tokens, sequence by sequence), then decode steps of all ten at once
    (projections at batch 10 on the GEMM, the attention stepping every
    sequence's kept state in one set of launches), then a step of the first
    three only (batch 3, the GEMV): every row against the oracle's block
    arithmetic on that sequence's own cache, to the block's tolerance."""
    from quantibbler_amd import DecoderBlock, FactorLayer

    d, H, Hk, hd, ffn, cap, blk = 256, 4, 2, 128, 512, 160, 64
    theta, eps = 500000.0, 1e-5
    lens = [0, 5, 70, 130, 1, 64, 0, 9, 33, 128]
    ns = len(lens)
    rng = np.random.default_rng(901)
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    bfv = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    norms = {"input": bfv(1.0 + 0.1 * rng.standard_normal(d)), "post_attention": bfv(1.0 + 0.1 * rng.standard_normal(d)),
             "q_norm": bfv(1.0 + 0.2 * rng.standard_normal(hd)), "k_norm": bfv(1.0 + 0.2 * rng.standard_normal(hd))}
    block = DecoderBlock(ctx, devs, norms["input"], norms["post_attention"], H, Hk, hd, theta, eps, cap, blk,
                         norms["q_norm"], norms["k_norm"], n_seqs=ns)
    st = torch.cuda.current_stream()
    kcs = [np.zeros((cap, Hk * hd), np.float32) for _ in range(ns)]
    vcs = [np.zeros((cap, Hk * hd), np.float32) for _ in range(ns)]
    for s, n in enumerate(lens):
        if n == 0:
            continue
        h = rng.standard_normal((n, d)).astype(np.float32)
        hdv = torch.from_numpy(h).cuda()
        wn = block.prefill_workspace_size(n)
        ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
        block.prefill_seq_dev(s, hdv, n, ws, wn, st)
        torch.cuda.synchronize()
        want = orc.block_prefill(layers, norms, h, kcs[s], vcs[s], H, Hk, hd, theta, eps)
        cos, rel = metrics(hdv.cpu().numpy(), want)
        assert cos >= COS_MIN and rel <= REL_MAX, (s, cos, rel)
    pos = list(lens)
    for n in (ns, ns, 3):
        x = rng.standard_normal((n, d)).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        wn = block.decode_batch_workspace_size(n)
        ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
        block.decode_batch_dev(xd, pos[:n], ws, wn, st)
        torch.cuda.synchronize()
        got = xd.cpu().numpy()
        for s in range(n):
            want = orc.block_step(layers, norms, x[s], pos[s], kcs[s], vcs[s], H, Hk, hd, theta, eps, "bf16",
                                  "sage", blk)
            cos, rel = metrics(got[s], want)
            print(f"batch {n}: sequence {s} at pos {pos[s]}: cos {cos:.7f} rel {rel:.2e}", flush=True)
            assert cos >= COS_MIN and rel <= REL_MAX, (n, s, pos[s], cos, rel)
        for s in range(n):
            pos[s] += 1
    # validation of the batched step
    from quantibbler_amd import KernelError

    h = torch.zeros((ns + 1) * d, dtype=torch.float32, device="cuda")
    ws = torch.empty(block.decode_batch_workspace_size(ns), dtype=torch.uint8, device="cuda")
    with pytest.raises(KernelError, match="batch of 11 sequences on a block holding 10"):
        block.decode_batch_dev(h, [0] * (ns + 1), ws, ws.numel(), st)
    with pytest.raises(KernelError, match=r"sequence 1: position 9 skips cache rows: the block holds 8 positions"):
        block.decode_batch_dev(h[:2 * d], [0, 9], ws, ws.numel(), st)
    with pytest.raises(KernelError, match="position 160 is past the block's cache capacity of 160"):
        block.decode_batch_dev(h[:d], [160], ws, ws.numel(), st)
    with pytest.raises(KernelError, match="workspace of 16 bytes is smaller"):
        block.decode_batch_dev(h[:d], [0], ws, 16, st)
    with pytest.raises(KernelError, match="sequence 10 of a block holding 10"):
        block.prefill_seq_dev(10, h[:d], 1, ws, ws.numel(), st)
    block.close()


@pytest.mark.parametrize("d,ffn", [(256, 512), (6144, 1024)])
def test_block_decode_fused_operands_bit_identical(ctx, orc, d, ffn):
    """The one-sequence step writes the projections' fp8 operands from its
    norm and SwiGLU kernels and adds the residual in the down projection's
    epilogue; the batched step at batch 1 runs the same arithmetic through
    separate prep and add kernels.  Two blocks of the same weights fed the
    same inputs stay bit-identical over 70 positions (a key-block boundary
    crossed); at d 6144 the set of three layers has 1152 operand runs, more
    than the norm's 1024 threads."""
    from quantibbler_amd import DecoderBlock, FactorLayer

    H, Hk, hd, cap, blk = 4, 2, 128, 80, 64
    theta, eps = 500000.0, 1e-5
    say(f"block fused operands d={d} ffn={ffn}")
    rng = np.random.default_rng(d + ffn)
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    bfv = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    norms = [bfv(1.0 + 0.1 * rng.standard_normal(d)), bfv(1.0 + 0.1 * rng.standard_normal(d))]
    qk = [bfv(1.0 + 0.2 * rng.standard_normal(hd)), bfv(1.0 + 0.2 * rng.standard_normal(hd))]
    one = DecoderBlock(ctx, devs, *norms, H, Hk, hd, theta, eps, cap, blk, *qk)
    bat = DecoderBlock(ctx, devs, *norms, H, Hk, hd, theta, eps, cap, blk, *qk, n_seqs=1)
    st = torch.cuda.current_stream()
    wn = bat.decode_batch_workspace_size(1)
    ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
    for pos in range(70):
        x = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
        ha, hb = x.clone(), x.clone()
        one.decode_dev(ha, pos, st)
        bat.decode_batch_dev(hb, [pos], ws, wn, st)
        torch.cuda.synchronize()
        assert torch.equal(ha, hb), (pos, float((ha - hb).abs().max()))


def test_block_batched_decode_many_sequences(ctx, orc):
    """32 sequences of 2 kv heads (64 (sequence, kv head) pairs: the
    attention pre-pass then runs one workgroup for K and one for V per pair
    and key block instead of splitting each four ways), prefilled to lengths
    across key-block boundaries, two batched steps: every row against the
    oracle's block arithmetic on that sequence's own cache."""
    from quantibbler_amd import DecoderBlock, FactorLayer

    d, H, Hk, hd, ffn, cap, blk = 256, 4, 2, 128, 512, 160, 64
    theta, eps = 500000.0, 1e-5
    ns = 32
    say(f"block batched decode, {ns} sequences")
    rng = np.random.default_rng(4242)
    lens = rng.integers(1, 140, ns).tolist()
    lens[:4] = [1, 63, 64, 128]
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    bfv = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    norms = {"input": bfv(1.0 + 0.1 * rng.standard_normal(d)), "post_attention": bfv(1.0 + 0.1 * rng.standard_normal(d)),
             "q_norm": bfv(1.0 + 0.2 * rng.standard_normal(hd)), "k_norm": bfv(1.0 + 0.2 * rng.standard_normal(hd))}
    block = DecoderBlock(ctx, devs, norms["input"], norms["post_attention"], H, Hk, hd, theta, eps, cap, blk,
                         norms["q_norm"], norms["k_norm"], n_seqs=ns)
    st = torch.cuda.current_stream()
    kcs = [np.zeros((cap, Hk * hd), np.float32) for _ in range(ns)]
    vcs = [np.zeros((cap, Hk * hd), np.float32) for _ in range(ns)]
    for s, n in enumerate(lens):
        h = rng.standard_normal((n, d)).astype(np.float32)
        hdv = torch.from_numpy(h).cuda()
        wn = block.prefill_workspace_size(n)
        ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
        block.prefill_seq_dev(s, hdv, n, ws, wn, st)
        torch.cuda.synchronize()
        orc.block_prefill(layers, norms, h, kcs[s], vcs[s], H, Hk, hd, theta, eps)
    pos = list(lens)
    wn = block.decode_batch_workspace_size(ns)
    ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
    for step in range(2):
        x = rng.standard_normal((ns, d)).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        block.decode_batch_dev(xd, pos, ws, wn, st)
        torch.cuda.synchronize()
        got = xd.cpu().numpy()
        worst = (1.0, 0.0)
        for s in range(ns):
            want = orc.block_step(layers, norms, x[s], pos[s], kcs[s], vcs[s], H, Hk, hd, theta, eps, "bf16",
                                  "sage", blk)
            cos, rel = metrics(got[s], want)
            worst = (min(worst[0], cos), max(worst[1], rel))
            assert cos >= COS_MIN and rel <= REL_MAX, (step, s, pos[s], cos, rel)
        say(f"step {step}: worst cos {worst[0]:.7f} rel {worst[1]:.2e}")
        pos = [p + 1 for p in pos]


def test_block_cache_written_by_the_caller(ctx, orc):
    """Cache rows written through qbk_block_cache and declared with
    qbk_block_set_filled: decoding continues at that position, the attention
    state rebuilt from the cache, bit-identical to a twin block that filled
    the same rows with its own prefill.  A device-position step is refused
    until an eager step has rebuilt the state (after the prefill as after
    set_filled), and accepted after it."""
    from quantibbler_amd import DecoderBlock, FactorLayer, KernelError

    d, H, Hk, hd, ffn, cap, blk = 256, 4, 2, 128, 512, 200, 64
    n = 70
    rng = np.random.default_rng(4711)
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    w_in = orc.bf16_round(1.0 + 0.1 * rng.standard_normal(d))
    w_post = orc.bf16_round(1.0 + 0.1 * rng.standard_normal(d))
    mk = lambda: DecoderBlock(ctx, devs, w_in, w_post, H, Hk, hd, 5e5, 1e-5, cap, blk)
    twin, ext = mk(), mk()
    st = torch.cuda.current_stream()
    say("caller-written cache: prefill the twin,", n, "tokens")
    h = torch.from_numpy(rng.standard_normal((n, d)).astype(np.float32)).cuda()
    wn = twin.prefill_workspace_size(n)
    ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
    twin.prefill_dev(h, n, ws, wn, st)
    pos_dev = torch.tensor([n], dtype=torch.int32, device="cuda")
    x = torch.zeros(d, dtype=torch.float32, device="cuda")
    with pytest.raises(KernelError, match="sequence 0: the attention state covers 0 of its 70 cached positions; "
                                          "a device-position step needs an eager step first"):
        twin.decode_pos_dev(x, pos_dev, st)
    # copy the twin's cache rows into the other block through the pointers
    def rows(ptr):
        # a torch view of the block's cache memory (the first n rows)
        sto = torch._C._construct_storage_from_data_pointer(ptr, torch.device("cuda", 0), n * Hk * hd * 4)
        return torch.empty(0, dtype=torch.float32, device="cuda").set_(sto, 0, (n, Hk * hd), (Hk * hd, 1))

    kt, vt = twin.cache_ptrs()
    ke, ve = ext.cache_ptrs()
    for src, dst in ((kt, ke), (vt, ve)):
        rows(dst).copy_(rows(src))
    torch.cuda.synchronize()
    with pytest.raises(KernelError, match=f"position {n} skips cache rows: the block holds 0 positions"):
        ext.decode_dev(x, n, st)
    ext.set_filled([n])
    with pytest.raises(KernelError, match="the attention state covers 0 of its 70 cached positions"):
        ext.decode_pos_dev(x, pos_dev, st)
    with pytest.raises(KernelError, match="201 rows exceed the block's cache capacity of 200"):
        ext.set_filled([cap + 1])
    for pos in range(n, n + 3):
        xin = rng.standard_normal(d).astype(np.float32)
        a = torch.from_numpy(xin).cuda()
        b = a.clone()
        twin.decode_dev(a, pos, st)
        ext.decode_dev(b, pos, st)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(a).all())
        assert torch.equal(a, b), f"position {pos}: caller-written cache differs from the twin's prefill"
    # the states now cover the cache: a device-position step is accepted
    pos_dev.fill_(n + 3)
    a = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
    b = a.clone()
    twin.decode_pos_dev(a, pos_dev, st)
    ext.decode_dev(b, n + 3, st)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    twin.close()
    ext.close()
