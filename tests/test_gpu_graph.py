"""GPU check: decode steps whose positions live in device memory
(qbk_block_decode_pos_dev, qbk_block_decode_batch_pos_dev,
qbk_positions_advance_dev), and those steps captured once in a HIP graph and
replayed at every later position.

The reference steps its engine from the host (engine/mod.rs:1377-1476); a
device-position step runs the same arithmetic as the eager step at that
position, so two blocks of the same weights fed the same inputs -- one
stepped eagerly, one by device positions or graph replays -- stay
bit-identical.  The runs cross key-block boundaries (64 tokens), where the
attention's kept state gains a block.  Graph replays are checked one by one
against the eager step, with eager work and synchronisations between them."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def scaled_layer(orc, rng, dout, din, r):
    ubs = rng.choice([-1, 1], (dout, r)).astype(np.int8)
    vts = rng.choice([-1, 1], (r, din)).astype(np.int8)
    s2 = np.exp(0.3 * rng.standard_normal(din)).astype(np.float32)
    s1 = (np.exp(0.3 * rng.standard_normal(dout)) / np.sqrt(r * din)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(dout)).astype(np.float32)
    return dict(dout=dout, din=din, r=r, ub=orc.pack_bits(ubs), vt=orc.pack_bits(vts), s1=s1, s2=s2,
                bias=bias)


def twin_blocks(ctx, orc, seed, H, Hk, n_seqs=None, d=256, hd=128, ffn=512, cap=200, blk=64):
    """Two blocks over the same device layers and norms."""
    from quantibbler_amd import DecoderBlock, FactorLayer

    rng = np.random.default_rng(seed)
    shapes = [(H * hd, d, 64), (Hk * hd, d, 32), (Hk * hd, d, 32), (d, H * hd, 64),
              (ffn, d, 96), (ffn, d, 96), (d, ffn, 96)]
    layers = [scaled_layer(orc, rng, *s) for s in shapes]
    devs = [FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                  L["bias"]) for L in layers]
    bfv = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32)))
    norms = [bfv(1.0 + 0.1 * rng.standard_normal(d)), bfv(1.0 + 0.1 * rng.standard_normal(d))]
    qk = [bfv(1.0 + 0.2 * rng.standard_normal(hd)), bfv(1.0 + 0.2 * rng.standard_normal(hd))]
    kw = {} if n_seqs is None else {"n_seqs": n_seqs}
    a = DecoderBlock(ctx, devs, *norms, H, Hk, hd, 500000.0, 1e-5, cap, blk, *qk, **kw)
    b = DecoderBlock(ctx, devs, *norms, H, Hk, hd, 500000.0, 1e-5, cap, blk, *qk, **kw)
    return a, b, devs, rng


@pytest.mark.parametrize("H,Hk", [(4, 1), (8, 2), (2, 2)])
def test_block_device_position_steps_bit_identical(ctx, orc, H, Hk):
    """Eager steps 0-4 on both blocks, then positions 5-134 by device
    position on one (the position advanced on the device after each step)
    and eagerly on the other; then the host record set and one more eager
    step on both."""
    from quantibbler_amd.gpu import advance_positions_dev

    say(f"device-position block steps H={H} Hk={Hk}")
    eag, dp, devs, rng = twin_blocks(ctx, orc, 900 + H + Hk, H, Hk)
    st = torch.cuda.current_stream()
    d = eag.d_model
    pos_dev = torch.zeros(1, dtype=torch.int32, device="cuda")
    for pos in range(5):
        x = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
        ha, hb = x.clone(), x.clone()
        eag.decode_dev(ha, pos, st)
        dp.decode_dev(hb, pos, st)
    pos_dev.fill_(5)
    for pos in range(5, 135):
        x = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
        ha, hb = x.clone(), x.clone()
        eag.decode_dev(ha, pos, st)
        dp.decode_pos_dev(hb, pos_dev, st)
        advance_positions_dev(ctx, pos_dev, 1, st)
        torch.cuda.synchronize()
        assert torch.equal(ha, hb), (pos, float((ha - hb).abs().max()))
    assert int(pos_dev.item()) == 135
    dp.set_positions([135])
    x = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
    ha, hb = x.clone(), x.clone()
    eag.decode_dev(ha, 135, st)
    dp.decode_dev(hb, 135, st)
    torch.cuda.synchronize()
    assert torch.equal(ha, hb)
    for blk in (eag, dp):
        blk.close()
    for L in devs:
        L.close()


@pytest.mark.parametrize("batched", [False, True])
def test_block_graph_replay_bit_identical(ctx, orc, batched):
    """One block step plus the position advance captured in a HIP graph
    (torch's graph API on ROCm), replayed 80 times across a key-block
    boundary: every replay's output equals the eager twin's step at that
    position.  The batched form steps three sequences at different
    positions (prefilled to 10, 63 and 64 tokens, then one eager step)."""
    from quantibbler_amd.gpu import advance_positions_dev

    say(f"graph replay of block steps, batched={batched}")
    n = 3 if batched else 1
    eag, dp, devs, rng = twin_blocks(ctx, orc, 77 + batched, 4, 1, n_seqs=n if batched else None)
    st = torch.cuda.current_stream()
    d = eag.d_model
    if batched:
        wn = eag.decode_batch_workspace_size(n)
        ws_a = torch.empty(wn, dtype=torch.uint8, device="cuda")
        ws_b = torch.empty(wn, dtype=torch.uint8, device="cuda")
        lens = [10, 63, 64]
        for s, m in enumerate(lens):
            h = torch.from_numpy(rng.standard_normal((m, d)).astype(np.float32)).cuda()
            pn = eag.prefill_workspace_size(m)
            pws = torch.empty(pn, dtype=torch.uint8, device="cuda")
            for blk in (eag, dp):
                hh = h.clone()
                blk.prefill_seq_dev(s, hh, m, pws, pn, st)
        pos = list(lens)
        x = torch.from_numpy(rng.standard_normal((n, d)).astype(np.float32)).cuda()
        ha, hb = x.clone(), x.clone()
        eag.decode_batch_dev(ha, pos, ws_a, wn, st)
        dp.decode_batch_dev(hb, pos, ws_b, wn, st)
        torch.cuda.synchronize()
        assert torch.equal(ha, hb)
        pos = [p + 1 for p in pos]
    else:
        for p in range(40):
            x = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
            ha, hb = x.clone(), x.clone()
            eag.decode_dev(ha, p, st)
            dp.decode_dev(hb, p, st)
        pos = [40]
    pos_dev = torch.tensor(pos, dtype=torch.int32, device="cuda")
    h_static = torch.zeros((n, d), dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        cs = torch.cuda.current_stream()
        if batched:
            dp.decode_batch_pos_dev(h_static, pos_dev, n, ws_b, wn, cs)
        else:
            dp.decode_pos_dev(h_static, pos_dev, cs)
        advance_positions_dev(ctx, pos_dev, n, cs)
    torch.cuda.synchronize()
    assert [int(v) for v in pos_dev.cpu()] == pos  # capture ran nothing
    for step in range(80):
        x = torch.from_numpy(rng.standard_normal((n, d)).astype(np.float32)).cuda()
        h_static.copy_(x)
        torch.cuda.synchronize()
        g.replay()
        ha = x.clone()
        if batched:
            eag.decode_batch_dev(ha, pos, ws_a, wn, st)
        else:
            eag.decode_dev(ha[0], pos[0], st)
        torch.cuda.synchronize()
        assert torch.equal(ha, h_static), (step, pos, float((ha - h_static).abs().max()))
        pos = [p + 1 for p in pos]
        assert [int(v) for v in pos_dev.cpu()] == pos
    del g
    for blk in (eag, dp):
        blk.close()
    for L in devs:
        L.close()


def test_block_device_position_past_capacity_skips(ctx, orc):
    """A device position at the capacity writes no cache row and steps no
    attention state (the kernels read the position and leave; the attention
    output is 0): after such a step the block continues eagerly,
    bit-identical to its twin that never took it."""
    from quantibbler_amd.gpu import advance_positions_dev

    say("device position at the capacity")
    eag, dp, devs, rng = twin_blocks(ctx, orc, 4711, 4, 1, cap=80)
    st = torch.cuda.current_stream()
    d = eag.d_model
    for pos in range(10):
        x = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
        ha, hb = x.clone(), x.clone()
        eag.decode_dev(ha, pos, st)
        dp.decode_dev(hb, pos, st)
    pos_dev = torch.tensor([80], dtype=torch.int32, device="cuda")
    junk = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
    dp.decode_pos_dev(junk, pos_dev, st)
    advance_positions_dev(ctx, pos_dev, 1, st)
    torch.cuda.synchronize()
    assert int(pos_dev.item()) == 81
    # the skipped attention reads as 0 (no key block), not 0/0: the step's
    # output stays finite
    assert bool(torch.isfinite(junk).all())
    for pos in range(10, 14):
        x = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).cuda()
        ha, hb = x.clone(), x.clone()
        eag.decode_dev(ha, pos, st)
        dp.decode_dev(hb, pos, st)
        torch.cuda.synchronize()
        assert torch.equal(ha, hb), (pos, float((ha - hb).abs().max()))
    for blk in (eag, dp):
        blk.close()
    for L in devs:
        L.close()
