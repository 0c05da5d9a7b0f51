#!/usr/bin/env python3
"""bench.py -- measure quantibbler-kernels' hot paths on one MI355X.

Headline (BASELINE.json metric, configs[0] shape): the binary-factor linear
decode GEMV, y = s1 . (Ub (Vb^T (s2 . x))), m = n = 4096, r = 1024, batch 1,
bf16 x and y, f32 accumulation, over a set of distinct layers (default 512,
537 MB of signs: larger than the 256 MB Infinity Cache, so HBM is what is
measured).  One step = one decode of every layer in the set: three launches
(the fp8 split of x; stage 1, t = bf16(Vb^T bf16(s2*x)), written as stage 2's
fp8 operand; stage 2, y = bf16(bf16(Ub t)*s1)).

value = algorithmic bytes of all layers / step time, with config 1's
per-layer count 1,097,728 B (U 512 KiB + V 512 KiB + x 8 KiB + y 8 KiB + s1,
s2 32 KiB).  The timed region holds only the steps between two events.  The
roofline's kernel duration: the timed step split by the kernels' shares,
which the same steps run again with an event between consecutive launches
measure (rocprofv3 --kernel-trace of the same command gives the kernels'
in-step durations; profiles/).

Extras (same JSON line): single-layer decode latency; prefill GEMM TFLOP/s at
B in {16, 128, 512, 2048}; block-scaled SageAttention prefill at
B=1, H=32, S=4096, d=128, causal; the reference scheme's decode
attention step at 4096 cached tokens (from scratch and on a kept state); the
lm_head at 128256 x 4096; one decoder block at config 3's shapes; config 5 at
batch 1 (a 2048-token prefill, then 256 greedy decode steps through 32 such
blocks, the final norm, the lm_head and argmax); config 3's
seven projections over 32 decoder layers (decode and prefill); and the CPU
baselines, each a bounded sample on the job's host CPUs (up to the 16-CPU
share of a one-GPU box): the headline's, the reference's bf16 serving
composite (apply_bf16 over the scalar core face) one layer per thread; the
reference fast face (fast.rs, f64x4, OpenMP over 64-row blocks) in the fp32
composite; the reference SageAttention scheme in f32 on two heads of config 4.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--layers 512]
    python bench.py --only gemm|sage|cfg3|sage_decode|head|block|model
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12          # B/s
BF16_PEAK = 2.5e15         # dense FLOP/s
INT8_PEAK = 5.0e15         # dense OP/s
LAYER_BYTES = 1_097_728    # config 1's algorithmic bytes per layer
M = N = 4096
R = 1024
METRIC = "factor-linear GB/s & %HBM peak (B=1); GEMM+SageAttn TFLOP/s & %MFMA peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemv_decode_config1_512layers.md")


def measured_traffic(stage):
    """HBM bytes per launch of a decode GEMV stage from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated against a copy
    kernel of known traffic), or None when the summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic-per-launch:"):
                    kv = dict(t.split("=") for t in line.split(":", 1)[1].split())
                    return int(kv[f"stage{stage}"])
    except (OSError, ValueError, KeyError):
        pass
    return None


def make_layers(qa, ctx, np, count, seed):
    rng = np.random.default_rng(seed)
    layers, host = [], []
    for i in range(count):
        ub = rng.integers(0, 256, (M, R // 8), dtype=np.uint8)
        vt = rng.integers(0, 256, (R, N // 8), dtype=np.uint8)
        s1 = np.exp(0.5 * rng.standard_normal(M)).astype(np.float32)
        s2 = np.exp(0.5 * rng.standard_normal(N)).astype(np.float32)
        layers.append(qa.FactorLayer.from_rows(ctx, M, N, R, ub, vt, s1, s2, None))
        if i < 16:
            host.append((ub, vt, s1, s2))
        if (i + 1) % 128 == 0:
            log(f"  uploaded {i + 1}/{count} layers")
    return layers, host


def bench_decode(qa, ctx, torch, np, layers, steps, warmup):
    """The timed region: `steps` decodes of the whole set (three launches
    each), bracketed by two events and nothing else.  Then the same steps
    again with an event between consecutive launches: each kernel's share of
    the step, which splits the timed step into the kernels' average
    durations (the roofline's denominator: the dominant kernel's)."""
    S = qa.FactorSet(ctx, layers)
    L = len(layers)
    rng = np.random.default_rng(7)
    xh = rng.standard_normal((L, N)).astype(np.float32)
    x = torch.from_numpy(xh).to("cuda").to(torch.bfloat16)
    y = torch.empty((L, M), dtype=torch.bfloat16, device="cuda")
    ws_n = S.workspace_size()
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    for _ in range(warmup):
        S.decode_dev(x, y, ws, ws_n, st)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(st)
    for _ in range(steps):
        S.decode_dev(x, y, ws, ws_n, st)
    end.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(end) / steps
    # each kernel's share of the step: the same steps again with an event
    # between consecutive launches on the launch stream; the shares split the
    # unperturbed step time above (an event adds a dispatch gap to the kernel
    # behind it, so the event intervals themselves run a few percent long)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(st)
        for ph in range(1, 4):
            S.stage_dev(ph, x, y, ws, ws_n, st)
            ev[i][ph].record(st)
    torch.cuda.synchronize()
    evt_ms = [sum(ev[i][ph - 1].elapsed_time(ev[i][ph]) for i in range(steps)) / steps for ph in range(1, 4)]
    phase_ms = [ms_step * e / sum(evt_ms) for e in evt_ms]
    return dict(ms_per_step=ms_step, phase_ms=phase_ms, evt_ms=evt_ms, wall_s=wall, set=S)


def bench_single_latency(torch, np, layer, iters=200):
    x = torch.randn((1, N), device="cuda").to(torch.bfloat16)
    y = torch.empty((1, M), dtype=torch.bfloat16, device="cuda")
    ws_n = layer.workspace_size(1)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    for _ in range(20):
        layer.linear_dev(x, 1, y, "bfloat16", ws, ws_n, st)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(iters):
        layer.linear_dev(x, 1, y, "bfloat16", ws, ws_n, st)
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters * 1e3  # us


def bench_gemm(torch, np, layer, batches=(16, 128, 512, 2048), iters=20):
    out = {}
    st = torch.cuda.current_stream()
    for B in batches:
        x = torch.randn((B, N), device="cuda").to(torch.bfloat16)
        y = torch.empty((B, M), dtype=torch.bfloat16, device="cuda")
        ws_n = layer.workspace_size(B)
        ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
        for _ in range(3):
            layer.linear_dev(x, B, y, "bfloat16", ws, ws_n, st)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(iters):
            layer.linear_dev(x, B, y, "bfloat16", ws, ws_n, st)
        b.record(st)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / iters
        flop = 2.0 * B * R * (M + N)
        tf = flop / (ms * 1e-3) / 1e12
        out[str(B)] = {"ms": round(ms, 4), "tflops": round(tf, 2), "frac_bf16_peak": round(tf * 1e12 / BF16_PEAK, 4)}
        log(f"  gemm B={B}: {ms:.3f} ms  {tf:.1f} TFLOP/s")
    return out


def bench_sage(qa, ctx, torch, np, iters=10):
    B, H, S, D = 1, 32, 4096, 128
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn((B, H, S, D), device="cuda", generator=g).to(torch.bfloat16)
    k = (torch.randn((B, H, S, D), device="cuda", generator=g)
         + 2.0 * torch.randn((B, H, 1, D), device="cuda", generator=g)).to(torch.bfloat16)
    v = torch.randn((B, H, S, D), device="cuda", generator=g).to(torch.bfloat16)
    o = torch.empty((B, H, S, D), dtype=torch.bfloat16, device="cuda")
    shape = qa.AttentionShape(B, H, H, S, S, D, D)
    ws_n = ctx.sage_blk_workspace_size(shape)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    for _ in range(3):
        ctx.attention_sage_blk_dev(shape, q, k, v, True, o, ws, ws_n, st)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(iters):
        ctx.attention_sage_blk_dev(shape, q, k, v, True, o, ws, ws_n, st)
    b.record(st)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / iters
    qk_ops = 2.0 * H * S * S * D / 2      # causal lower triangle, int8
    pv_flops = 2.0 * H * S * S * D / 2    # fp16
    blended_peak = (qk_ops + pv_flops) / (qk_ops / INT8_PEAK + pv_flops / BF16_PEAK)
    tops = (qk_ops + pv_flops) / (ms * 1e-3)
    log(f"  sage blk cfg4: {ms:.3f} ms  {tops / 1e12:.1f} TOPS blended")
    return {"ms": round(ms, 4), "tops_blended": round(tops / 1e12, 2),
            "frac_blended_peak": round(tops / blended_peak, 4),
            "blended_peak_tops": round(blended_peak / 1e12, 1),
            "shape": "B=1 H=32 S=4096 d=128 causal, bf16 in/out, includes the quantisation pre-pass"}


def bench_sage_decode(qa, ctx, torch, np, seq=4096, iters=20):
    """One decode step of the reference scheme (engine/mod.rs:984-1030) over a
    row-major f32 KV cache at config 3's attention shape (32 query heads,
    8 kv heads, d = 128, block 64): the O(seq) step, and the reference's own
    call pattern (the query in row 0 of a zero-padded seq-row problem,
    causal=False, the cache gathered head-major) on the same device."""
    H, Hk, D, block = 32, 8, 128, 64
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn((H, D), device="cuda", generator=g)
    k = torch.randn((seq, Hk, D), device="cuda", generator=g) + 2.0 * torch.randn((1, Hk, D), device="cuda", generator=g)
    v = torch.randn((seq, Hk, D), device="cuda", generator=g)
    o = torch.empty((H, D), dtype=torch.float32, device="cuda")
    sh = qa.AttentionShape(1, H, Hk, 1, seq, D, D)
    wn = ctx.sage_decode_workspace_size(sh, block)
    ws = torch.empty(wn, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    def step():
        ctx.attention_sage_decode_dev(sh, q, k, v, block, o, ws, wn, st)
    for _ in range(5):
        step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(iters):
        step()
    b.record(st)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / iters
    cache_bytes = seq * Hk * 2 * D * 4
    # the same step in a decode loop on a kept state: the cache grew by one
    # token since the state's last step, so only the last key block is
    # quantised again
    cap = seq + 64
    sn = qa.SageDecodeState.size(ctx, H, Hk, D, D, cap, block)
    sws = torch.empty(sn, dtype=torch.uint8, device="cuda")
    oc = torch.empty_like(o)
    ctx.attention_sage_decode_step_dev(sh, q, k, v, block, oc, sws, sn, cap, 0, st)
    def kept():
        ctx.attention_sage_decode_step_dev(sh, q, k, v, block, oc, sws, sn, cap, seq - 1, st)
    for _ in range(5):
        kept()
    torch.cuda.synchronize()
    a.record(st)
    for _ in range(iters):
        kept()
    b.record(st)
    torch.cuda.synchronize()
    kept_ms = a.elapsed_time(b) / iters
    kept_same = bool(torch.equal(oc, o))
    # the reference's call pattern, timed once after a warm-up call (its
    # gather and padding counted as free)
    qp = torch.zeros((1, H, seq, D), device="cuda")
    qp[0, :, 0, :] = q
    kp = k.permute(1, 0, 2).contiguous()[None]
    vp = v.permute(1, 0, 2).contiguous()[None]
    op = torch.empty((1, H, seq, D), device="cuda")
    shp = qa.AttentionShape(1, H, Hk, seq, seq, D, D)
    ctx.attention_sage_dev(shp, qp, kp, vp, False, block, op, st)
    torch.cuda.synchronize()
    a.record(st)
    ctx.attention_sage_dev(shp, qp, kp, vp, False, block, op, st)
    b.record(st)
    torch.cuda.synchronize()
    pad_ms = a.elapsed_time(b)
    same = bool(torch.equal(op[0, :, 0, :], o))
    log(f"  sage decode seq={seq}: {ms * 1e3:.1f} us/step ({cache_bytes / (ms * 1e-3) / 1e9:.0f} GB/s of cache); "
        f"padded reference call {pad_ms:.2f} ms; row 0 identical: {same}; on a kept state "
        f"{kept_ms * 1e3:.1f} us/step (identical: {kept_same})")
    return {"us_per_step": round(ms * 1e3, 1), "kept_state_us_per_step": round(kept_ms * 1e3, 1),
            "kept_state_bit_identical": kept_same, "cache_bytes": cache_bytes,
            "GB/s": round(cache_bytes / (ms * 1e-3) / 1e9, 1),
            "padded_reference_call_ms": round(pad_ms, 3), "row0_bit_identical": same,
            "shape": f"H=32 Hkv=8 d=128 seq={seq} block 64, f32 row-major cache"}


def bench_head(qa, ctx, torch, np, vocab=128256, d=4096, iters=20):
    """The language-model head of config 5 (engine/mod.rs:781-800): one
    decode step's logits over a bf16-valued 128256 x 4096 head (1.05 GB
    stored as bf16, the bytes that dominate a batch-1 decode step), and
    batches of 8 and 32 positions (config 5's batch; bit-exact sequential
    sums, so bound by the vector ALU: 2 * 32 * 128256 * 4096 f32 operations)."""
    g = torch.Generator(device="cuda").manual_seed(11)
    rows = torch.randn((vocab, d), device="cuda", generator=g).to(torch.bfloat16).to(torch.float32)
    H = qa.LmHead.from_rows_dev(ctx, rows, vocab, d)
    del rows
    torch.cuda.empty_cache()
    hid = torch.randn((32, d), device="cuda", generator=g).to(torch.bfloat16).to(torch.float32)
    out = torch.empty((32, vocab), dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream()
    res = {"vocab": vocab, "d_model": d, "stored_bf16": H.bf16, "head_bytes": vocab * d * 2}
    for b in (1, 8, 32):
        for _ in range(3):
            H.logits_dev(hid, b, out, st)
        torch.cuda.synchronize()
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(iters):
            H.logits_dev(hid, b, out, st)
        e.record(st)
        torch.cuda.synchronize()
        ms = a.elapsed_time(e) / iters
        res[f"batch{b}_us"] = round(ms * 1e3, 1)
        res[f"batch{b}_GB/s"] = round(vocab * d * 2 / (ms * 1e-3) / 1e9, 1)
        log(f"  lm_head batch {b}: {ms * 1e3:.1f} us, {vocab * d * 2 / (ms * 1e-3) / 1e9:.0f} GB/s")
    H.close()
    return res


# the seven projections of a Llama-3-8B-shaped
# decoder layer, ranks from the reference's planning rule at 0.55 bits/weight
# (v2 stream, fp16 scales): (name, dout, din, r).
CFG3 = [("q", 4096, 4096, 1102), ("k", 1024, 4096, 431), ("v", 1024, 4096, 431),
        ("o", 4096, 4096, 1102), ("gate", 14336, 4096, 1724), ("up", 14336, 4096, 1724),
        ("down", 4096, 14336, 1733)]
# bytes of one decoder layer's seven v2 streams (qpk1 lib.rs:152-210): a
# 24-byte header, fp16 s1 (dout), s2 (din) and bias (dout), then the two
# continuous sign bitstreams -- 14,995,624 B
CFG3_REF_LAYER_BYTES = sum(24 + 2 * (2 * m + n) + (m * r + 7) // 8 + (n * r + 7) // 8 for _, m, n, r in CFG3)


def random_rows(np, rng, n_rows, n_bits):
    """Random +-1 rows, packed LSB-first with zero pad bits."""
    b = rng.integers(0, 256, (n_rows, (n_bits + 7) // 8), dtype=np.uint8)
    if n_bits % 8:
        b[:, -1] &= (1 << (n_bits % 8)) - 1
    return b


def bench_block(qa, ctx, torch, np, ctx_tokens=2048, steps=50):
    """One decoder block of config 3 (engine/mod.rs:878-945: norm, q/k/v,
    RoPE, cache append, the sage decode attention on a kept state, o +
    residual, norm, gate/up, SwiGLU, down + residual) at one position, with
    ctx_tokens already in its cache: time per block per token, and that
    times 32 for the trunk of a 32-block model.  Scales keep activations
    near unit size (s1 ~ 1/sqrt(r din))."""
    rng = np.random.default_rng(44)
    layers = []
    for name, m, n, r in CFG3:
        s1 = (np.exp(0.3 * rng.standard_normal(m)) / np.sqrt(r * n)).astype(np.float32)
        s2 = np.exp(0.3 * rng.standard_normal(n)).astype(np.float32)
        layers.append(qa.FactorLayer.from_rows(ctx, m, n, r, random_rows(np, rng, m, r),
                                               random_rows(np, rng, r, n), s1, s2, None))
    d = 4096
    w_in = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    w_post = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    B = qa.DecoderBlock(ctx, layers, w_in, w_post, 32, 8, 128, 500000.0, 1e-5, ctx_tokens + steps + 64, 64)
    st = torch.cuda.current_stream()
    hs = torch.randn((ctx_tokens + steps, d), device="cuda")
    for pos in range(ctx_tokens):  # fill the cache, one position a call
        B.decode_dev(hs[pos], pos, st)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for pos in range(ctx_tokens, ctx_tokens + steps):
        B.decode_dev(hs[pos], pos, st)
    b.record(st)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / steps * 1e3
    finite = bool(torch.isfinite(hs[ctx_tokens:]).all())
    B.close()
    log(f"  decoder block (config 3 shapes) at {ctx_tokens}-{ctx_tokens + steps} cached tokens: "
        f"{us:.1f} us per block per token, x32 = {32 * us / 1e3:.2f} ms")
    return {"us_per_block_token": round(us, 1), "trunk_32_blocks_ms": round(32 * us / 1e3, 3),
            "cached_tokens": ctx_tokens, "outputs_finite": finite,
            "shape": "d 4096, 32/8 heads x 128, ffn 14336, config-3 ranks; bf16 serving, sage decode attention"}


def bench_model(qa, ctx, torch, np, n_blocks=32, prompt=2048, steps=256, vocab=128256, batches=(1, 32)):
    """Config 5, all on the device: a random-init 32-block Llama-3-8B-shaped
    model at config 3's ranks (each block its own layers, 480 MB of signs in
    all, and per sequence its own KV cache), an embedding of 128256 rows,
    fp16-valued norms, and a 128256 x 4096 bf16 lm_head.  Workload per batch
    size b: the prefill of `prompt` random token ids into each of b sequences
    (every block's one-pass prefill: projections on the GEMM at batch
    `prompt`, causal block-scaled SageAttention), the last positions' logits
    and greedy tokens, then `steps` greedy decode steps of all b sequences
    together (embedding rows, 32 DecoderBlocks -- projections at batch b, the
    sage decode attention stepping each sequence's kept state -- final norm,
    logits, argmax; engine/mod.rs:802-822, :1377-1476, sampler.rs:4-15), the
    next tokens fed back on the device.  Each batch size runs twice: with
    the steps launched from the host, and (after a second prefill and one
    host-launched step) with the step captured once in a HIP graph --
    device positions, advanced on the device -- and replayed `steps` - 1
    times."""
    from quantibbler_amd.gpu import advance_positions_dev, argmax_dev, embed, embed_dev, rms_norm_dev

    rng = np.random.default_rng(55)
    d = 4096
    nseq = max(batches)
    cap = prompt + steps + 64
    blocks, keep = [], []
    for bi in range(n_blocks):
        layers = []
        for name, m, n, r in CFG3:
            s1 = (np.exp(0.3 * rng.standard_normal(m)) / np.sqrt(r * n)).astype(np.float16).astype(np.float32)
            s2 = np.exp(0.3 * rng.standard_normal(n)).astype(np.float16).astype(np.float32)
            layers.append(qa.FactorLayer.from_rows(ctx, m, n, r, random_rows(np, rng, m, r),
                                                   random_rows(np, rng, r, n), s1, s2, None))
        w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float16).astype(np.float32)
        blocks.append(qa.DecoderBlock(ctx, layers, w, w, 32, 8, 128, 500000.0, 1e-5, cap, 64, n_seqs=nseq))
        keep.append(layers)
        if (bi + 1) % 8 == 0:
            log(f"  config 5: built {bi + 1}/{n_blocks} blocks ({nseq} sequences' caches each)")
    g = torch.Generator(device="cuda").manual_seed(56)
    rows = (0.02 * torch.randn((vocab, d), device="cuda", generator=g)).to(torch.bfloat16).to(torch.float32)
    head = qa.LmHead.from_rows_dev(ctx, rows, vocab, d)
    del rows
    table = torch.randn((vocab, d), device="cuda", generator=g).to(torch.bfloat16).to(torch.float32)
    w_final = torch.ones(d, dtype=torch.float32, device="cuda")
    logits = torch.empty((nseq, vocab), dtype=torch.float32, device="cuda")
    h = torch.empty((nseq, d), dtype=torch.float32, device="cuda")
    hn = torch.empty((nseq, d), dtype=torch.float32, device="cuda")
    tok = torch.zeros(nseq, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream()
    ids = rng.integers(0, vocab, (nseq, prompt)).astype(np.int32)
    hp = torch.empty((prompt, d), dtype=torch.float32, device="cuda")
    wn = max(B.prefill_workspace_size(prompt) for B in blocks)
    wd = max(B.decode_batch_workspace_size(b) for B in blocks for b in batches)
    ws = torch.empty(max(wn, wd), dtype=torch.uint8, device="cuda")

    def prefill(b):
        for B in blocks:
            B.reset()
        for sq in range(b):
            embed(ctx, table, vocab, d, ids[sq], hp, st)
            for B in blocks:
                B.prefill_seq_dev(sq, hp, prompt, ws, wn, st)
            rms_norm_dev(ctx, hp[prompt - 1], 1, d, w_final, 1e-5, hn[sq], st)
        head.logits_dev(hn, b, logits, st)
        argmax_dev(ctx, logits, b, vocab, tok, st)

    def token(b, pos):
        embed_dev(ctx, table, vocab, d, tok, b, h, st)
        if b == 1:
            for B in blocks:
                B.decode_dev(h[0], pos, st)
        else:
            p = [pos] * b
            for B in blocks:
                B.decode_batch_dev(h, p, ws, wd, st)
        rms_norm_dev(ctx, h, b, d, w_final, 1e-5, hn, st)
        head.logits_dev(hn, b, logits, st)
        argmax_dev(ctx, logits, b, vocab, tok, st)

    pos_dev = torch.zeros(nseq, dtype=torch.int32, device="cuda")

    def token_dev(b, s):
        # the same step with the positions in pos_dev, advanced at its end
        embed_dev(ctx, table, vocab, d, tok, b, h, s)
        if b == 1:
            for B in blocks:
                B.decode_pos_dev(h[0], pos_dev, s)
        else:
            for B in blocks:
                B.decode_batch_pos_dev(h, pos_dev, b, ws, wd, s)
        rms_norm_dev(ctx, h, b, d, w_final, 1e-5, hn, s)
        head.logits_dev(hn, b, logits, s)
        argmax_dev(ctx, logits, b, vocab, tok, s)
        advance_positions_dev(ctx, pos_dev, b, s)

    out = {}
    prefill(1)          # warm-up pass (first launches, allocator)
    token(1, prompt)
    torch.cuda.synchronize()
    for b in batches:
        a, e1, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        a.record(st)
        prefill(b)
        e1.record(st)
        for i in range(steps):
            token(b, prompt + i)
        c.record(st)
        torch.cuda.synchronize()
        pre_ms, dec_ms = a.elapsed_time(e1), e1.elapsed_time(c) / steps
        finite = bool(torch.isfinite(logits[:b]).all())
        log(f"  config 5 (B={b}): prefill of {b} x {prompt} tokens {pre_ms:.2f} ms, then {steps} greedy steps "
            f"at {dec_ms:.3f} ms/step ({b * 1e3 / dec_ms:.1f} tokens/s)")
        eager_tok = tok[:b].clone()
        # the graph-replayed loop: prefill again, one host-launched step
        # (the attention states then hold every complete key block), the
        # step captured once, then replayed for the remaining steps
        prefill(b)
        token(b, prompt)
        pos_dev[:b] = prompt + 1
        side = torch.cuda.Stream()
        side.wait_stream(st)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            token_dev(b, torch.cuda.current_stream())
        torch.cuda.synchronize()
        a.record(st)
        for i in range(steps - 1):
            graph.replay()
        c.record(st)
        torch.cuda.synchronize()
        graph_ms = a.elapsed_time(c) / (steps - 1)
        same_tokens = bool(torch.equal(tok[:b], eager_tok))
        del graph
        for B in blocks:
            B.set_positions([prompt + steps] * b)
        log(f"  config 5 (B={b}): graph-replayed steps at {graph_ms:.3f} ms/step ({b * 1e3 / graph_ms:.1f} "
            f"tokens/s), final tokens {'equal to' if same_tokens else 'DIFFERENT from'} the host-launched loop's")
        out[f"b{b}"] = {"batch": b, "prefill_ms": round(pre_ms, 2),
                        "prefill_tokens_per_s": round(b * prompt / pre_ms * 1e3, 1),
                        "decode_ms_per_step": round(dec_ms, 3),
                        "decode_tokens_per_s": round(b * 1e3 / dec_ms, 1),
                        "graph_decode_ms_per_step": round(graph_ms, 3),
                        "graph_decode_tokens_per_s": round(b * 1e3 / graph_ms, 1),
                        "graph_tokens_equal": same_tokens,
                        "prompt_tokens": prompt, "decode_steps": steps, "logits_finite": finite}
    for B in blocks:
        B.close()
    head.close()
    out["shape"] = ("32 blocks (d 4096, 32/8 heads x 128, ffn 14336, config-3 ranks, fp16-valued scales), "
                    "embedding and lm_head 128256 x 4096, bf16 serving; prefill on the GEMM and the "
                    "block-scaled SageAttention, decode on the GEMV (batch 1) or the GEMM (batch 32) and "
                    "the sage decode attention")
    return out


def bench_cfg3(qa, ctx, torch, np, n_layers=32, steps=100, prefill_b=2048):
    """Decode (batch 1) of every projection of n_layers distinct decoder
    layers -- 480 MB of signs, beyond the 256 MB MALL -- as one FactorSet
    over all of them (three launches per token); then the prefill GEMM of
    one layer's projections at B = prefill_b."""
    rng = np.random.default_rng(33)
    groups, ordered = {}, []
    sign_bytes = act_bytes = 0
    for li in range(n_layers):
        for name, m, n, r in CFG3:
            # fp16 scales (configs[2]: "packed signs plus fp16 scales"), which the
            # decode streams as fp16
            L = qa.FactorLayer.from_rows(ctx, m, n, r, random_rows(np, rng, m, r), random_rows(np, rng, r, n),
                                         np.exp(0.5 * rng.standard_normal(m)).astype(np.float16).astype(np.float32),
                                         np.exp(0.5 * rng.standard_normal(n)).astype(np.float16).astype(np.float32),
                                         None)
            groups.setdefault((m, n, r), []).append(L)
            ordered.append(L)
            sign_bytes += (m * r + 7) // 8 + (n * r + 7) // 8
            act_bytes += 2 * n + 2 * m + 2 * m + 2 * n  # x, y (bf16), s1, s2 (fp16)
        if (li + 1) % 8 == 0:
            log(f"  cfg3: uploaded {li + 1}/{n_layers} decoder layers")
    st = torch.cuda.current_stream()
    # one set over every projection of every layer, in decoder-layer order
    # (q, k, v, o, gate, up, down of layer 0, then layer 1, ...): three
    # launches per token
    all_layers = ordered
    S = qa.FactorSet(ctx, all_layers)
    n_in = sum(L.din for L in all_layers)
    n_out = sum(L.dout for L in all_layers)
    x = torch.randn(n_in, device="cuda").to(torch.bfloat16)
    y = torch.empty(n_out, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(S.workspace_size(), dtype=torch.uint8, device="cuda")
    def token():
        S.decode_dev(x, y, ws, ws.numel(), st)
    for _ in range(100):  # ~10 ms: the clocks settle (3 tokens read ~10 % slow)
        token()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(steps):
        token()
    b.record(st)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    total = sign_bytes + act_bytes
    ref = n_layers * CFG3_REF_LAYER_BYTES
    out = {"decoder_layers": n_layers, "sign_bytes": sign_bytes, "ref_bytes_per_token": ref,
           "ms_per_token": round(ms, 4), "GB/s": round(ref / (ms * 1e-3) / 1e9, 1),
           "frac_hbm_peak": round(ref / (ms * 1e-3) / HBM_PEAK, 4),
           "bytes_streamed_per_token": total,
           "bytes_note": "frac and GB/s count the reference's v2 streams (signs + fp16 s1/s2/bias, "
                         "14,995,624 B a decoder layer); bytes_streamed_per_token is what this "
                         "build reads (signs, fp16 s1 and s2, bf16 x and y; the bias is zero and not read)"}
    log(f"  cfg3 decode: {ms:.3f} ms/token over {n_layers} layers, {out['GB/s']} GB/s")
    # prefill: one decoder layer's seven projections at B = prefill_b
    flop = 0
    calls = []
    for name, m, n, r in CFG3:
        L = groups[(m, n, r)][0]
        xb = torch.randn((prefill_b, n), device="cuda").to(torch.bfloat16)
        yb = torch.empty((prefill_b, m), dtype=torch.bfloat16, device="cuda")
        wn = L.workspace_size(prefill_b)
        wsb = torch.empty(wn, dtype=torch.uint8, device="cuda")
        calls.append((L, xb, yb, wsb, wn))
        flop += 2.0 * prefill_b * r * (m + n)
    def layer():
        for L, xb, yb, wsb, wn in calls:
            L.linear_dev(xb, prefill_b, yb, "bfloat16", wsb, wn, st)
    layer()
    torch.cuda.synchronize()
    a.record(st)
    for _ in range(5):
        layer()
    b.record(st)
    torch.cuda.synchronize()
    pms = a.elapsed_time(b) / 5
    tf = flop / (pms * 1e-3) / 1e12
    out["prefill"] = {"B": prefill_b, "ms_per_layer": round(pms, 3), "gflop": round(flop / 1e9, 1),
                      "tflops": round(tf, 1), "frac_bf16_peak": round(tf * 1e12 / BF16_PEAK, 4)}
    log(f"  cfg3 prefill B={prefill_b}: {pms:.3f} ms/layer, {tf:.1f} TFLOP/s")
    return out


def host_info():
    """The host the CPU baselines ran on: CPU model, logical CPUs, the CPUs
    this process may use, and the oracle's compiler flags."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    flags = ""
    try:
        with open(os.path.join(ROOT, "oracle", "Makefile")) as f:
            for line in f:
                if line.startswith("CFLAGS"):
                    flags = line.split("=", 1)[1].strip()
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    return {"cpu_model": model, "nproc": os.cpu_count(), "cpus_allowed": allowed,
            "compiler": "gcc " + flags}


def cpu_threads():
    """Threads for the CPU baselines: every CPU this process may use, capped
    at the 16-CPU share a one-GPU box grants a job."""
    info = host_info()
    return max(1, min(16, info["cpus_allowed"]))


def bench_cpu(np, host, budget_s=10.0):
    """The headline's CPU baseline: the reference's bf16 serving composite
    (engine/mod.rs:449-460 apply_bf16 over the scalar core face,
    core.rs:202-260, as the reference serves bf16 on the CPU) on the decode
    workload's independent layers, one layer per thread at a time on every
    thread of the job's CPU share, for about budget_s seconds."""
    from concurrent.futures import ThreadPoolExecutor

    from oracle import oracle as orc

    orc.build()
    threads = cpu_threads()
    rng = np.random.default_rng(11)
    x = rng.standard_normal(N).astype(np.float32)

    def one(i):
        ub, vt, s1, s2 = host[i % len(host)]
        orc.factor_apply("bf16", M, N, R, ub, vt, s1, s2, None, x)

    calls, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        while time.perf_counter() - t0 < budget_s:
            list(pool.map(one, range(calls, calls + threads)))
            calls += threads
    dt = time.perf_counter() - t0
    out = {"value": round(calls * LAYER_BYTES / dt / 1e9, 4), "unit": "GB/s", "cores": threads,
           "kind": "port",
           "sample": f"{calls} bf16-serving decode calls of config-1 layers (m=n=4096, r=1024, B=1) "
                     f"cycling {len(host)} distinct layers in {dt:.1f} s, one layer per thread: the "
                     "oracle's C restatement of apply_bf16 (engine/mod.rs:449-460) over the scalar "
                     "core face (core.rs:202-260)"}
    out.update(host_info())
    return out


def bench_cpu_fast(np, host, budget_s=5.0):
    """The reference's fastest CPU face, fast.rs:28-110 (f64x4 lanes, 64-row
    tasks over every thread) inside the fp32 serving composite
    (engine/mod.rs:393-437), on the same layers."""
    from oracle import oracle as orc

    threads = cpu_threads()
    rng = np.random.default_rng(12)
    x = rng.standard_normal(N).astype(np.float32)
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        ub, vt, s1, s2 = host[calls % len(host)]
        orc.factor_apply("fp32", M, N, R, ub, vt, s1, s2, None, x, fast=True, threads=threads)
        calls += 1
    dt = time.perf_counter() - t0
    return {"value": round(calls * LAYER_BYTES / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{calls} fp32-serving decode calls in {dt:.1f} s (fast face, f64x4, OpenMP)"}


def bench_cpu_sage(np, heads=2, seq=4096):
    """The reference SageAttention scheme in f32 (gpu_attention.rs:89-396
    semantics, the oracle's restatement, OpenMP over query rows) on a bounded
    sample of config 4: `heads` of its 32 heads at its full sequence, causal,
    block 64; reported as config 4's operation rate (per head: 2 S^2 d / 2
    INT8 ops + the same in P.V)."""
    from oracle import oracle as orc

    threads = cpu_threads()
    rng = np.random.default_rng(13)
    q = rng.standard_normal((1, heads, seq, 128)).astype(np.float32)
    k = (rng.standard_normal((1, heads, seq, 128)) + 2 * rng.standard_normal((1, heads, 1, 128))).astype(np.float32)
    v = rng.standard_normal((1, heads, seq, 128)).astype(np.float32)
    t0 = time.perf_counter()
    orc.attention_sage_dev(q, k, v, True, 64, threads=threads)
    dt = time.perf_counter() - t0
    ops = heads * 2 * (2 * seq * seq * 128 / 2)
    return {"value": round(ops / dt / 1e12, 5), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"{heads} heads x {seq} tokens x d 128, causal, block 64 in {dt:.1f} s "
                      f"({dt / heads * 32:.0f} s for config 4's 32 heads)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=512)
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--only", choices=["gemm", "sage", "cfg3", "sage_decode", "head", "block", "model"],
                    help="run one secondary workload alone and print its figures (for profiling); "
                         "no headline line")
    ap.add_argument("--model-steps", type=int, default=256, help="config 5's greedy decode steps")
    ap.add_argument("--model-batches", default="1,32", help="config 5's batch sizes, comma-separated")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate-traffic", action="store_true",
                    help="first run an elementwise kernel of known traffic (256 MiB read, 256 MiB "
                         "written) that rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs scale by")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(one process drives one GPU; this build runs no collectives)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import quantibbler_amd as qa

    ctx = qa.GpuContext(0)
    if args.calibrate_traffic:
        a = torch.ones(1 << 26, dtype=torch.int32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            torch.neg(a, out=b)
        torch.cuda.synchronize()
        del a, b
    if args.only:
        if args.only == "gemm":
            layers, _ = make_layers(qa, ctx, np, 1, seed=1)
            res = bench_gemm(torch, np, layers[0])
        elif args.only == "sage":
            res = bench_sage(qa, ctx, torch, np)
        elif args.only == "sage_decode":
            res = bench_sage_decode(qa, ctx, torch, np)
        elif args.only == "head":
            res = bench_head(qa, ctx, torch, np)
        elif args.only == "block":
            res = bench_block(qa, ctx, torch, np)
        elif args.only == "model":
            res = bench_model(qa, ctx, torch, np, steps=args.model_steps,
                              batches=tuple(int(b) for b in args.model_batches.split(",")))
        else:
            res = bench_cfg3(qa, ctx, torch, np)
        print(json.dumps({"only": args.only, "result": res}), flush=True)
        return
    log(f"building {args.layers} config-1 layers ...")
    layers, host = make_layers(qa, ctx, np, args.layers, seed=1)
    log("decode sweep ...")
    d = bench_decode(qa, ctx, torch, np, layers, args.steps, args.warmup)
    total_bytes = args.layers * LAYER_BYTES
    value = total_bytes / (d["ms_per_step"] * 1e-3) / 1e9
    ph = d["phase_ms"]
    # algorithmic bytes per layer of each GEMV kernel: stage 1 streams Vb
    # (r x n bits; the prep carries x and s2), stage 2 streams Ub (m x r bits)
    # and reads s1, writes y
    gemv_bytes = {1: N * R // 8, 2: M * R // 8 + 4 * M + 2 * M}
    dom = 1 if ph[1] >= ph[2] else 2
    dom_ms = ph[1] if dom == 1 else ph[2]
    bytes_launch = args.layers * gemv_bytes[dom]
    achieved = bytes_launch / (dom_ms * 1e-3) / 1e9
    log(f"  decode: {d['ms_per_step']:.3f} ms/step, {value:.1f} GB/s; phases (prep x, gemv 1 + "
        f"t operand, gemv 2) = {', '.join(f'{p:.4f}' for p in ph)} ms")
    ev = d["evt_ms"]
    extra = {"decode_phase_ms": {"prep_x": round(ph[0], 4), "gemv_stage1": round(ph[1], 4),
                                 "gemv_stage2": round(ph[2], 4)},
             "decode_phase_event_interval_ms": {"prep_x": round(ev[0], 4), "gemv_stage1": round(ev[1], 4),
                                                "gemv_stage2": round(ev[2], 4)}}
    if not args.no_extra:
        log("single-layer latency ...")
        extra["decode_single_layer_us"] = round(bench_single_latency(torch, np, layers[0]), 2)
        log("prefill GEMM ...")
        extra["prefill_gemm"] = bench_gemm(torch, np, layers[0])
        log("sage attention ...")
        extra["sage_blk"] = bench_sage(qa, ctx, torch, np)
        log("sage decode step ...")
        extra["sage_decode"] = bench_sage_decode(qa, ctx, torch, np)
        log("lm_head ...")
        extra["lm_head"] = bench_head(qa, ctx, torch, np)
        extra["decoder_block"] = bench_block(qa, ctx, torch, np)
        log("config 5: prefill + greedy decode (32 blocks + lm_head) ...")
        extra["config5"] = bench_model(qa, ctx, torch, np, steps=args.model_steps,
                                       batches=tuple(int(b) for b in args.model_batches.split(",")))
        log("config 3 (8B decoder layer projections) ...")
        extra["cfg3_8b_layer"] = bench_cfg3(qa, ctx, torch, np)
    log("cpu baseline ...")
    cpu = bench_cpu(np, host, args.cpu_seconds)
    if not args.no_extra:
        log("cpu baselines: fast face, reference sage scheme ...")
        extra["cpu_fast_face_f64"] = bench_cpu_fast(np, host)
        extra["cpu_sage_reference_f32"] = bench_cpu_sage(np)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"decode GEMV (batch 1) over {args.layers} distinct config-1 factor layers "
                        "(m=n=4096, r=1024, +-1 Bernoulli(0.5) signs, lognormal(0,0.5) fp32 scales, "
                        "bf16 N(0,1) x), one launch per stage for the whole set",
            "layers": args.layers, "m": M, "n": N, "r": R, "batch": 1,
            "weight_bytes": args.layers * (M * R + N * R) // 8,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": round(achieved / (HBM_PEAK / 1e9), 4), "traffic": measured_traffic(dom),
            "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT),
            "kernel": f"q4_gemv_kernel<{dom},*,2> (decode stage {dom}, fp4 x fp8 scaled MFMA)",
            "bytes_per_launch": bytes_launch, "avg_launch_ms": round(dom_ms, 4),
            "avg_launch_source": "the timed step (two HIP events on the launch stream) times the "
                                 "kernel's share of the step, measured over the same steps run again "
                                 "with an event between consecutive launches",
            "event_interval_ms": round(d["evt_ms"][dom], 4),
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
