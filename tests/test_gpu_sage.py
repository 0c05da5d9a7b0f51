"""GPU parity: SageAttention through the C ABI.

Reference scheme (gpu_attention.rs:589-756): on every attention_sage.json
case the device output is bit-identical to the oracle's f32 restatement of
the reference kernel, passes the reference's device gate against the f64
quantized reference (gpu_attention_sage.rs:35-46), and stays inside its
measured quality envelope against exact attention.

Block-scaled scheme: INT8 codes and scales bit-identical to the oracle's
pre-pass; outputs within 1 bf16 ulp-scale tolerance of the oracle; quality
against exact attention at cos >= 0.999, relL1 <= 0.02.
"""
import numpy as np
import pytest

from conftest import load_golden, same
from test_oracle_attention import COS_MIN, RL1_MAX, SLACK, dense_attention, metrics, shaped, two_part_gate

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def say(*a):
    print(*a, flush=True)


def shape_of(q, k, v):
    from quantibbler_amd import AttentionShape

    b, h, s, d = q.shape
    return AttentionShape(b, h, k.shape[1], s, s, d, v.shape[3])


def test_reference_scheme_fixture_battery(ctx, orc):
    for rec in load_golden("attention_sage.json"):
        q, k, v = (shaped(rec, n, t) for n, t in (("query", "q"), ("key", "k"), ("value", "v")))
        say("sage ref fixture", rec["seed"], rec["shape"], rec["causal"], rec["block_size"])
        out = ctx.attention_sage(shape_of(q, k, v), q, k, v, rec["causal"], rec["block_size"])
        want = orc.attention_sage_dev(q, k, v, rec["causal"], rec["block_size"])
        same(out, want.ravel())
        two_part_gate(out, rec["faces"]["quantized-reference"]["out"], rec["shape"]["val_dim"])
        cos, rl1 = metrics(out, rec["faces"]["exact"]["out"])
        ref = rec["reference_metrics"]
        assert cos >= COS_MIN and rl1 <= RL1_MAX
        assert cos >= ref["cosine"] - SLACK and rl1 <= ref["relative_l1"] + SLACK


def padded_decode_call(ctx, qh, kc, vc, block):
    """engine/mod.rs:984-1030 gqa_attention_sage as the reference makes it: the
    step's query in row 0 of a zero-padded (pos + 1)-row problem, the cache
    gathered head-major (KvCache::head_major, engine/mod.rs:1258-1268),
    attention_sage with causal=False, row 0 of each head read back."""
    from quantibbler_amd import AttentionShape

    h, d = qh.shape
    seq, hk, dv = vc.shape
    q = np.zeros((1, h, seq, d), np.float32)
    q[0, :, 0, :] = qh
    k = np.ascontiguousarray(kc.transpose(1, 0, 2))[None]
    v = np.ascontiguousarray(vc.transpose(1, 0, 2))[None]
    out = ctx.attention_sage(AttentionShape(1, h, hk, seq, seq, d, dv), q, k, v, False, block)
    return out.reshape(h, seq, dv)[:, 0, :], (q, k, v)


@pytest.mark.parametrize("h,hk,d,dv,seq,block", [
    (4, 2, 16, 16, 1, 1), (4, 2, 16, 16, 37, 8), (8, 2, 64, 64, 200, 64), (4, 1, 128, 128, 130, 64),
    (2, 1, 32, 48, 150, 100), (8, 8, 128, 128, 333, 64), (4, 2, 64, 64, 90, 256),
    (2, 1, 6, 10, 45, 16),   # channels not a multiple of 4: the general pre-pass
    (32, 2, 128, 128, 129, 64),   # 16 heads a kv head
    (8, 2, 128, 128, 75, 16), (4, 1, 32, 32, 70, 64),   # four heads a kv head: short blocks, short heads
    # more than 512 blocks: the running max scanned first (per-head kernels;
    # two scan passes past 2048 blocks; grouped kernels)
    (2, 1, 16, 16, 1100, 2), (2, 1, 16, 16, 4200, 2), (4, 2, 64, 64, 8400, 16),
])
def test_decode_step_matches_padded_reference_call(ctx, orc, h, hk, d, dv, seq, block):
    """One decode step over a row-major KV cache: bit-identical to row 0 of the
    reference's padded call, both on this device and in the oracle."""
    from quantibbler_amd import AttentionShape

    say("sage decode step", h, hk, d, dv, seq, block)
    rng = np.random.default_rng(7 * seq + block + h)
    qh = rng.standard_normal((h, d)).astype(np.float32)
    kc = (rng.standard_normal((seq, hk, d)) + 2.0 * rng.standard_normal((1, hk, d))).astype(np.float32)
    vc = rng.standard_normal((seq, hk, dv)).astype(np.float32)
    sh = AttentionShape(1, h, hk, 1, seq, d, dv)
    got = ctx.attention_sage_decode(sh, qh, kc, vc, block)
    want_dev, (q, k, v) = padded_decode_call(ctx, qh, kc, vc, block)
    same(got, want_dev)
    if seq * seq * d * h <= 2e9:  # the oracle's padded call is O(seq^2)
        want = orc.attention_sage_dev(q, k, v, False, block)[0, :, 0, :]
        same(got, want)
    # the device-pointer form, twice on one workspace
    wn = ctx.sage_decode_workspace_size(sh, block)
    ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
    qd, kd, vd = (torch.from_numpy(a).cuda() for a in (qh, kc, vc))
    od = torch.empty((h, dv), dtype=torch.float32, device="cuda")
    for _ in range(2):
        ctx.attention_sage_decode_dev(sh, qd, kd, vd, block, od, ws, wn, torch.cuda.current_stream())
        torch.cuda.synchronize()
        same(od.cpu().numpy(), got)


@pytest.mark.parametrize("h,hk,d,dv,block,steps", [
    (4, 2, 64, 64, 16, [1, 2, 15, 16, 17, 18, 31, 32, 33, 60, 61, 64, 65, 100]),
    (8, 2, 128, 128, 64, [1, 63, 64, 65, 66, 127, 128, 129, 200, 255, 256, 257]),
    (2, 1, 32, 48, 100, [5, 99, 100, 101, 150, 230]),   # blocks wider than one LDS chunk
])
def test_decode_state_steps_match_fresh_calls(ctx, orc, h, hk, d, dv, block, steps):
    """A decode loop over a growing cache on one kept state (only the blocks
    from the last complete one on quantised again): every step bit-identical
    to a fresh call; a reset state on a different cache starts over."""
    from quantibbler_amd import AttentionShape, KernelError, SageDecodeState

    say("sage decode state", h, hk, d, dv, block, steps[-1])
    cap = steps[-1] + 7
    rng = np.random.default_rng(11 * block + h)
    kc = (rng.standard_normal((cap, hk, d)) + 2.0 * rng.standard_normal((1, hk, d))).astype(np.float32)
    vc = rng.standard_normal((cap, hk, dv)).astype(np.float32)
    kd, vd = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    size = SageDecodeState.size(ctx, h, hk, d, dv, cap, block)
    with pytest.raises(KernelError, match="decode state of .* bytes is smaller than the"):
        SageDecodeState(ctx, h, hk, d, dv, cap, block, torch.empty(size - 1, dtype=torch.uint8, device="cuda"))
    st = SageDecodeState(ctx, h, hk, d, dv, cap, block, torch.empty(size, dtype=torch.uint8, device="cuda"))
    od = torch.empty((h, dv), dtype=torch.float32, device="cuda")
    for i, seq in enumerate(steps):
        qh = rng.standard_normal((h, d)).astype(np.float32)
        st.step(torch.from_numpy(qh).cuda(), kd, vd, seq, od, torch.cuda.current_stream())
        torch.cuda.synchronize()
        sh = AttentionShape(1, h, hk, 1, seq, d, dv)
        want = ctx.attention_sage_decode(sh, qh, kc[:seq], vc[:seq], block)
        same(od.cpu().numpy(), want)
        if i % 5 == 4:
            q = np.zeros((1, h, seq, d), np.float32)
            q[0, :, 0, :] = qh
            k = np.ascontiguousarray(kc[:seq].transpose(1, 0, 2))[None]
            v = np.ascontiguousarray(vc[:seq].transpose(1, 0, 2))[None]
            same(od.cpu().numpy(), orc.attention_sage_dev(q, k, v, False, block)[0, :, 0, :])
    # a new sequence in the same cache buffers: the kept codes are stale
    kc2 = rng.standard_normal((cap, hk, d)).astype(np.float32)
    kd.copy_(torch.from_numpy(kc2))
    st.reset()
    qh = rng.standard_normal((h, d)).astype(np.float32)
    seq = steps[len(steps) // 2]
    st.step(torch.from_numpy(qh).cuda(), kd, vd, seq, od, torch.cuda.current_stream())
    torch.cuda.synchronize()
    same(od.cpu().numpy(), ctx.attention_sage_decode(AttentionShape(1, h, hk, 1, seq, d, dv), qh, kc2[:seq],
                                                      vc[:seq], block))
    # a shorter cache than the last step's starts over by itself
    seq2 = max(1, seq - block - 1)
    st.step(torch.from_numpy(qh).cuda(), kd, vd, seq2, od, torch.cuda.current_stream())
    torch.cuda.synchronize()
    same(od.cpu().numpy(), ctx.attention_sage_decode(AttentionShape(1, h, hk, 1, seq2, d, dv), qh,
                                                      kc2[:seq2], vc[:seq2], block))


@pytest.mark.parametrize("b,h,hk,s,d,dv,causal,block", [
    (1, 4, 2, 200, 64, 64, True, 64),
    (2, 2, 1, 130, 128, 128, True, 64),
    (1, 2, 2, 96, 32, 48, False, 16),
    (1, 2, 1, 150, 16, 16, True, 100),   # blocks wider than one LDS chunk
    (1, 1, 1, 70, 8, 8, False, 70),
])
def test_reference_scheme_random_bit_identical(ctx, orc, b, h, hk, s, d, dv, causal, block):
    say("sage ref random", b, h, hk, s, d, dv, causal, block)
    rng = np.random.default_rng(s + d + block)
    q = rng.standard_normal((b, h, s, d)).astype(np.float32)
    k = (rng.standard_normal((b, hk, s, d)) + 2 * rng.standard_normal((b, hk, 1, d))).astype(np.float32)
    v = rng.standard_normal((b, hk, s, dv)).astype(np.float32)
    out = ctx.attention_sage(shape_of(q, k, v), q, k, v, causal, block)
    want = orc.attention_sage_dev(q, k, v, causal, block)
    same(out, want.ravel())
    # Against the f64 NumPy semantics the f32 scheme differs wherever an INT8
    # code lands on the other side of a rounding boundary (the reference's
    # 1e-4 gate is pinned on its fixture battery only), so the f64 form is a
    # quality comparison here, as is exact attention.
    npref = orc.attention_sage_np(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), causal, block)
    c, r = metrics(out, npref)
    assert c > 0.99999 and r < 2e-3, (c, r)
    c, r = metrics(out, dense_attention(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), causal))
    assert c >= COS_MIN and r <= RL1_MAX, (c, r)


def test_reference_scheme_device_pointer_form(ctx, orc):
    say("sage ref dev form")
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 2, 64, 32)).astype(np.float32)
    k = rng.standard_normal((1, 1, 64, 32)).astype(np.float32)
    v = rng.standard_normal((1, 1, 64, 32)).astype(np.float32)
    sh = shape_of(q, k, v)
    qd, kd, vd = (torch.from_numpy(a).cuda() for a in (q, k, v))
    od = torch.empty((1, 2, 64, 32), dtype=torch.float32, device="cuda")
    ctx.attention_sage_dev(sh, qd, kd, vd, True, 8, od, torch.cuda.current_stream())
    torch.cuda.synchronize()
    same(od.cpu().numpy(), orc.attention_sage_dev(q, k, v, True, 8))


def run_blk(ctx, qb, kb, vb, causal):
    sh = shape_of(qb, kb, vb)
    qd, kd, vd = (torch.from_numpy(a.view(np.int16)).cuda() for a in (qb, kb, vb))
    od = torch.empty(qb.shape[:3] + (vb.shape[3],), dtype=torch.int16, device="cuda")
    ws_n = ctx.sage_blk_workspace_size(sh)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    ctx.attention_sage_blk_dev(sh, qd, kd, vd, causal, od, ws, ws_n, torch.cuda.current_stream())
    torch.cuda.synchronize()
    return od.cpu().numpy().view(np.uint16)


def blk_inputs(orc, rng, b, h, hk, s):
    q = rng.standard_normal((b, h, s, 128)).astype(np.float32)
    k = (rng.standard_normal((b, hk, s, 128)) + 2 * rng.standard_normal((b, hk, 1, 128))).astype(np.float32)
    v = rng.standard_normal((b, hk, s, 128)).astype(np.float32)
    return tuple(orc.f32_to_bf16_fast(a) for a in (q, k, v))


@pytest.mark.parametrize("b,h,hk,s", [(1, 2, 2, 64), (1, 4, 2, 200), (2, 2, 1, 333), (1, 2, 1, 1024)])
def test_blk_prepass_codes_bit_identical(ctx, orc, b, h, hk, s):
    say("sage blk prepass", b, h, hk, s)
    rng = np.random.default_rng(b * 100 + s)
    qb, kb, vb = blk_inputs(orc, rng, b, h, hk, s)
    _, st = orc.attention_sage_blk(qb, kb, vb, causal=True, stages=True)
    sh = shape_of(qb, kb, vb)
    nblk = (s + 63) // 64
    qd, kd, vd = (torch.from_numpy(a.view(np.int16)).cuda() for a in (qb, kb, vb))
    qh = torch.empty((b, h, s, 128), dtype=torch.int8, device="cuda")
    kh = torch.empty((b, hk, s, 128), dtype=torch.int8, device="cuda")
    qs = torch.empty((b, h, nblk), dtype=torch.float32, device="cuda")
    ks = torch.empty((b, hk, nblk), dtype=torch.float32, device="cuda")
    km = torch.empty((b, hk, 128), dtype=torch.float32, device="cuda")
    vh = torch.empty((b, hk, s, 128), dtype=torch.int16, device="cuda")
    ctx.sage_blk_quantize_dev(sh, qd, kd, vd, qh, qs, kh, ks, km, vh, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert np.array_equal(qh.cpu().numpy(), st["qhat"])
    assert np.array_equal(kh.cpu().numpy(), st["khat"])
    same(qs.cpu().numpy(), st["qscale"])
    same(ks.cpu().numpy(), st["kscale"])
    same(km.cpu().numpy(), st["kmean"])
    vf = orc.bf16_to_f32(vb)
    assert np.array_equal(vh.cpu().numpy().view(np.float16).astype(np.float32), vf.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("b,h,hk,s,causal", [
    (1, 2, 2, 64, True), (1, 4, 2, 200, True), (2, 2, 1, 333, False), (1, 2, 1, 1024, True),
    (1, 2, 2, 128, False),
])


def test_blk_attention_against_oracle_and_exact(ctx, orc, b, h, hk, s, causal):
    say("sage blk attention", b, h, hk, s, causal)
    rng = np.random.default_rng(b * 1000 + s + causal)
    qb, kb, vb = blk_inputs(orc, rng, b, h, hk, s)
    got = orc.bf16_to_f32(run_blk(ctx, qb, kb, vb, causal)).astype(np.float64)
    want = orc.attention_sage_blk(qb, kb, vb, causal=causal).astype(np.float64)
    # outputs are bf16: allow 2 bf16 ulps of each value plus a row-scale floor
    rowmax = np.abs(want).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - want) <= 2 ** -7 * np.abs(want) + 2e-3 * rowmax)
    c, r = metrics(got, want)
    assert c > 0.99999 and r < 4e-3
    exact = dense_attention(*(orc.bf16_to_f32(a).astype(np.float64) for a in (qb, kb, vb)), causal)
    c, r = metrics(got, exact)
    assert c >= COS_MIN and r <= RL1_MAX, (c, r)
    again = orc.bf16_to_f32(run_blk(ctx, qb, kb, vb, causal)).astype(np.float64)
    same(again, got)

def test_blk_attention_config4_full_size_quality(ctx):
    """Config 4 at its full shape (B = 1, H = 32, S = 4096, d = 128, causal,
    K with a per-channel offset of std 2): every output finite, the run
    deterministic, and rows sampled across the sequence within the quality
    gate of exact attention (cos >= 0.999, relL1 <= 0.02), the exact rows
    computed on the device in fp32."""
    import math

    from quantibbler_amd import AttentionShape

    say("sage blk config 4 full size")
    B, H, S, D = 1, 32, 4096, 128
    g = torch.Generator(device="cuda").manual_seed(44)
    q = torch.randn((B, H, S, D), device="cuda", generator=g).to(torch.bfloat16)
    k = (torch.randn((B, H, S, D), device="cuda", generator=g)
         + 2.0 * torch.randn((B, H, 1, D), device="cuda", generator=g)).to(torch.bfloat16)
    v = torch.randn((B, H, S, D), device="cuda", generator=g).to(torch.bfloat16)
    sh = AttentionShape(B, H, H, S, S, D, D)
    wn = ctx.sage_blk_workspace_size(sh)
    ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(2):
        o = torch.empty((B, H, S, D), dtype=torch.bfloat16, device="cuda")
        ctx.attention_sage_blk_dev(sh, q, k, v, True, o, ws, wn, torch.cuda.current_stream())
        torch.cuda.synchronize()
        outs.append(o)
    assert torch.equal(outs[0], outs[1])
    got = outs[0].float()
    assert bool(torch.isfinite(got).all())
    rows = torch.tensor([0, 1, 63, 64, 65, 127, 1000, 2047, 2048, 3333, 4095], device="cuda")
    qf, kf, vf = q.float(), k.float(), v.float()
    cos_min, rl1_max = 1.0, 0.0
    for h in range(H):
        sc = torch.matmul(qf[0, h, rows], kf[0, h].t().contiguous()) / math.sqrt(D)
        keep = torch.arange(S, device="cuda")[None, :] <= rows[:, None]
        sc = sc.masked_fill(~keep, float("-inf"))
        want = torch.matmul(torch.softmax(sc, dim=-1), vf[0, h]).double().cpu().numpy()
        have = got[0, h, rows].double().cpu().numpy()
        c, r = metrics(have, want)
        cos_min, rl1_max = min(cos_min, c), max(rl1_max, r)
    say("  cos_min", cos_min, "rl1_max", rl1_max)
    assert cos_min >= COS_MIN and rl1_max <= RL1_MAX, (cos_min, rl1_max)


def test_blk_attention_closed_forms(ctx, orc):
    """Cases whose block-scaled output is fixed by the mathematics, not by the
    oracle: (i) every key equal -> every score 0, p = 1, row i = mean of V
    over keys 0..i; (ii) one key scoring more than 150 (log2 units) above the
    rest -> every other p underflows, the output row is that key's V row
    exactly (rows from it on; causal rows of the first key block are case
    (i) again)."""
    say("sage blk closed forms")
    rng = np.random.default_rng(9330)
    s = 192
    q = rng.standard_normal((1, 2, s, 128)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 1, 1, 128)).astype(np.float32), s, axis=2)
    v = rng.standard_normal((1, 1, s, 128)).astype(np.float32)
    qb, kb, vb = (orc.f32_to_bf16_fast(a) for a in (q, k, v))
    vf = orc.bf16_to_f32(vb).astype(np.float64)[0, 0]
    for causal in (True, False):
        got = orc.bf16_to_f32(run_blk(ctx, qb, kb, vb, causal)).astype(np.float64)
        mean = (np.cumsum(vf, axis=0) / np.arange(1, s + 1)[:, None]) if causal else \
            np.broadcast_to(vf.mean(axis=0), (s, 128))
        for h in range(2):
            assert np.all(np.abs(got[0, h] - mean) <= 2 ** -8 * np.abs(mean) + 1e-6), (causal, h)
    star = 150
    q = np.zeros((1, 1, s, 128), np.float32)
    q[..., 0] = 64.0
    k = np.zeros((1, 1, s, 128), np.float32)
    k[0, 0, :, 0] = -1.0
    k[0, 0, star, 0] = 60.0
    qb, kb = orc.f32_to_bf16_fast(q), orc.f32_to_bf16_fast(k)
    got = orc.bf16_to_f32(run_blk(ctx, qb, kb, vb[:, :1], False))[0, 0]
    assert np.array_equal(got, np.broadcast_to(orc.bf16_to_f32(vb)[0, 0, star], (s, 128)))
    got = orc.bf16_to_f32(run_blk(ctx, qb, kb, vb[:, :1], True))[0, 0].astype(np.float64)
    assert np.array_equal(got[star:], np.broadcast_to(vf[star], (s - star, 128)))
    mean = np.cumsum(vf, axis=0) / np.arange(1, s + 1)[:, None]
    assert np.all(np.abs(got[:64] - mean[:64]) <= 2 ** -8 * np.abs(mean[:64]) + 1e-6)
