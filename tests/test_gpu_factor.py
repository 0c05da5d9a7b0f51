"""GPU parity: the binary factor linear (engine/mod.rs:393-481) through the C
ABI against the oracle.

* Integer-exact inputs (small-integer z, so every f32 sum is exact and every
  bf16 rounding is decided by the exact value): the device composite must be
  bit-identical to the oracle's -- a single misplaced bit anywhere in the
  repacked layouts would change an output.
* Config-distribution inputs: each stage within the reference's bf16 backward
  bound (1e-2 of the row term scale, parity.rs:797-806 and
  engine/mod.rs:1897-1949), and within one bf16 ulp of the oracle's stage
  output (the two differ only by f32 reassociation).
"""
import numpy as np
import pytest

from conftest import same

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def say(*a):
    print(*a, flush=True)


def make_layer(orc, rng, dout, din, r, integer=False):
    ubs = rng.choice([-1, 1], (dout, r)).astype(np.int8)
    vts = rng.choice([-1, 1], (r, din)).astype(np.int8)
    if integer:
        s2 = np.ones(din, np.float32)
    else:
        s2 = np.exp(0.5 * rng.standard_normal(din)).astype(np.float32)
    s1 = np.exp(0.5 * rng.standard_normal(dout)).astype(np.float32)
    bias = rng.standard_normal(dout).astype(np.float32)
    return dict(dout=dout, din=din, r=r, ub=orc.pack_bits(ubs), vt=orc.pack_bits(vts), s1=s1,
                s2=s2, bias=bias, ubs=ubs, vts=vts)


def upload(ctx, L):
    from quantibbler_amd import FactorLayer

    return FactorLayer.from_rows(ctx, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"],
                                 L["s2"], L["bias"])


def run_dev(layer, x_bf16, y_dtype="float32"):
    batch = x_bf16.shape[0]
    x = torch.from_numpy(x_bf16.view(np.int16)).cuda()
    y = torch.empty((batch, layer.dout), dtype=torch.float32 if y_dtype == "float32" else torch.int16,
                    device="cuda")
    ws_n = layer.workspace_size(batch)
    ws = torch.zeros(ws_n, dtype=torch.uint8, device="cuda")
    layer.linear_dev(x, batch, y, y_dtype, ws, ws_n, torch.cuda.current_stream())
    torch.cuda.synchronize()
    yy = y.cpu().numpy()
    if y_dtype == "bfloat16":
        yy = yy.view(np.uint16)
    return yy, ws.cpu().numpy()


SHAPES = [(256, 512, 128), (300, 200, 37), (1024, 4096, 1102), (4096, 4096, 1024)]


@pytest.mark.parametrize("dout,din,r", SHAPES)
@pytest.mark.parametrize("batch", [1, 2, 8, 9, 16, 32, 33, 128])
def test_integer_exact_bit_identical(ctx, orc, dout, din, r, batch):
    integer_exact_case(ctx, orc, dout, din, r, batch)


@pytest.mark.parametrize("dout,din,r", [(4096, 14336, 1733), (512, 9000, 200)])
def test_integer_exact_long_k_batch1(ctx, orc, dout, din, r):
    """A lone layer of long K at batch 1 (config 3's down projection, and a
    K that is not a multiple of 128): stage 1 splits each row group's slices
    over eight waves (512-thread workgroups) instead of four."""
    integer_exact_case(ctx, orc, dout, din, r, 1)


@pytest.mark.parametrize("dout,din,r,batch", [(300, 200, 37, 1031), (256, 512, 128, 1024), (1024, 4096, 1102, 1024),
                                              (512, 640, 2000, 1030), (301, 200, 37, 1031), (1030, 384, 100, 1024)])
def test_integer_exact_one_launch(ctx, orc, dout, din, r, batch):
    """The one-launch GEMM (batches from 256 on): ragged last token groups,
    a din that is not a multiple of 128, ranks whose 64-row groups do not
    split evenly over the eight waves (1102: 18 groups), and the largest rank
    it takes (2000: 32 groups, four a wave).  A dout that is not a multiple
    of 4 (301, 1030) runs the element-wise y stores, a kernel of its own."""
    integer_exact_case(ctx, orc, dout, din, r, batch)


@pytest.mark.parametrize("batch", [255, 512])
def test_integer_exact_config2_mid_batches(ctx, orc, batch):
    """Config 2's shape at B = 255 (the two-stage GEMM's largest batch: the
    K-split stage 1 on 128 x 64 tiles, stage 2 on its own 256 tiles) and B =
    512 (the one-launch GEMM on 64 workgroups)."""
    integer_exact_case(ctx, orc, 4096, 4096, 1024, batch)


def integer_exact_case(ctx, orc, dout, din, r, batch):
    say("factor integer-exact", dout, din, r, "batch", batch)
    rng = np.random.default_rng(dout + din + r + batch)
    L = make_layer(orc, rng, dout, din, r, integer=True)
    layer = upload(ctx, L)
    x = orc.f32_to_bf16_fast(rng.integers(-2, 3, (batch, din)).astype(np.float32))
    want = orc.factor_apply_bf16_batch(dout, din, r, L["ub"], L["vt"], L["s1"], L["s2"], L["bias"], x)
    got, _ = run_dev(layer, x)
    same(got, want)
    got_b, _ = run_dev(layer, x, "bfloat16")
    same(got_b, orc.f32_to_bf16_fast(want))


def test_prefill_gemm_config2_full_size_integer_exact(ctx, orc):
    """Config 2 at its largest batch (m = n = 4096, r = 1024, B = 2048) on
    integer-exact inputs (s2 = 1, x in {-2..2}): the expectation is formed on
    the device by fp32 products of the unpacked +-1 factors, exact for these
    integers in any summation order (|t| <= 8192, |u| < 2^24), with the bf16
    roundings of t and u and the final s1 / bias in separate fp32 operations,
    as engine/mod.rs:449-460 does them."""
    say("factor full-size prefill B=2048 integer-exact")
    rng = np.random.default_rng(2048)
    dout = din = 4096
    r, batch = 1024, 2048
    L = make_layer(orc, rng, dout, din, r, integer=True)
    layer = upload(ctx, L)
    x = orc.f32_to_bf16_fast(rng.integers(-2, 3, (batch, din)).astype(np.float32))
    got, _ = run_dev(layer, x)
    got_b, _ = run_dev(layer, x, "bfloat16")
    xf = torch.from_numpy(orc.bf16_to_f32(x)).cuda()
    vt_t = torch.from_numpy(L["vts"].astype(np.float32).T.copy()).cuda()   # (din, r)
    u_t = torch.from_numpy(L["ubs"].astype(np.float32).T.copy()).cuda()    # (r, dout)
    t = torch.matmul(xf, vt_t).to(torch.bfloat16).float()
    u = torch.matmul(t, u_t).to(torch.bfloat16).float()
    y = u * torch.from_numpy(L["s1"]).cuda()
    y = y + torch.from_numpy(L["bias"]).cuda()
    want = y.cpu().numpy()
    same(got, want, "f32 out")
    same(got_b, orc.f32_to_bf16_fast(want), "bf16 out")


def e4m3(b):
    """OCP fp8 e4m3 bytes -> float64 (bias 7, subnormals, no infinities)."""
    b = np.asarray(b, np.uint8).astype(np.int64)
    e, m = (b >> 3) & 0xF, b & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7))
    return np.where(b & 0x80, -v, v)


def kq4(g, e):
    """k offset within a 128-slice of fp4 element e of lane group g (gfx950
    scaled MFMA, measured): two runs of 16."""
    return 16 * (g >> 1) + 64 * (g & 1) + (e & 15) + 32 * (e >> 4)


def gpu_t(layer, ws, batch):
    """The device's t (bf16) read back from the documented workspace layout."""
    r, rp = layer.r, -(-layer.r // 128) * 128
    rnd = lambda n: -(-n // 256) * 256
    if batch <= 32:
        # fp4 decode (the factor linear's route up to 32 tokens):
        # [op1 | sc1 | op2 [slice][4][ncol][32] | sc2 [slice][4][ncol]]:
        # t is stage 2's operand, hi (column 2b) + lo (2b+1), E8M0 scales
        ns1, ns2, ncol = -(-layer.din // 128), rp // 128, 2 * batch
        o2 = rnd(ns1 * 4 * ncol * 32) + rnd(ns1 * 4 * ncol)
        op = ws[o2: o2 + ns2 * 4 * ncol * 32].reshape(ns2, 4, ncol, 32)
        sc = ws[o2 + rnd(ns2 * 4 * ncol * 32):][: ns2 * 4 * ncol].reshape(ns2, 4, ncol).astype(np.int64)
        t = np.zeros((batch, rp))
        for g in range(4):
            for e in range(32):
                gb, byte, k = 2 * (g & 1) + (e >> 4), 16 * (g >> 1) + (e & 15), kq4(g, e)
                for b in range(batch):
                    hi = e4m3(op[:, gb, 2 * b, byte]) * 2.0 ** (sc[:, g, 2 * b] - 127)
                    lo = e4m3(op[:, gb, 2 * b + 1, byte]) * 2.0 ** (sc[:, g, 2 * b + 1] - 127)
                    t[b, np.arange(ns2) * 128 + k] = hi + lo
        from oracle import oracle as orc

        tb = orc.f32_to_bf16_fast(t.astype(np.float32))
        assert np.array_equal(orc.bf16_to_f32(tb).astype(np.float64), t), "operand is not a bf16 t"
        assert not tb[:, r:].any()
        return tb[:, :r]
    if ws.size == batch * rp * 2:
        # fused prefill GEMM (gemm.hip): t bf16 [batch][r_p], zero past r
        t = ws.view(np.uint16).reshape(batch, rp)
        assert not t[:, r:].any()
        return t[:, :r]
    # two-stage prefill GEMM (rank past 2048): [z bf16 [batch][din_p] | f32 partials [split][batch][r_p]
    # (split > 1) | t bf16 [batch][r_p] | stage 2's f32 partials
    # [split2][batch][dout_p] (split2 > 1)]
    from oracle import oracle as orc

    zb = rnd(batch * (-(-layer.din // 64) * 64) * 2)
    dp = -(-layer.dout // 128) * 128
    sizes = {(s, s2) for s in (1, 2, 4, 8) for s2 in (1, 2, 4, 8)}
    for s, s2 in sorted(sizes):
        pb = rnd(s * batch * rp * 4) if s > 1 else 0
        p2 = rnd(s2 * batch * dp * 4) if s2 > 1 else 0
        if zb + pb + rnd(batch * rp * 2) + p2 == ws.size:
            t = ws[zb + pb: zb + pb + batch * rp * 2].view(np.uint16).reshape(batch, rp)
            assert not t[:, r:].any()
            if s > 1:
                parts = ws[zb: zb + s * batch * rp * 4].view(np.float32).reshape(s, batch, rp)
                tot = parts[0].copy()
                for i in range(1, s):
                    tot = (tot + parts[i]).astype(np.float32)
                assert np.array_equal(orc.f32_to_bf16_fast(tot[:, :r]), t[:, :r])
            return t[:, :r]
    raise AssertionError("unexpected workspace size")


def mfma_window(v):
    """Bound on what the fp4 x fp8 scaled MFMA's own summation can lose in a
    stage fed v [batch][K]: the MFMA sums each 32-element scale block (the
    runs kq4(g, .) of a 128-k slice) in a fixed-point window about 13 bits
    below the block's largest product, truncating what falls below it (probed
    on gfx950 with planted operands: one large product and small ones in the
    same block lose bits, across blocks nothing is lost); measured losses stay
    under 2^-10 of the block's largest product.  v's hi piece carries the
    block maximum, its lo piece at most 2^-4 of it, and the epilogue divides
    out the 1.5 of the fp4 signs: per token, 2^-10 (1 + 2^-4) times the sum
    of the blocks' largest |v|."""
    v = np.abs(np.asarray(v, np.float64))
    K = v.shape[1]
    kp = -(-K // 128) * 128
    w = np.zeros((v.shape[0], kp))
    w[:, :K] = v
    k = np.arange(kp) % 128
    grp = (np.arange(kp) // 128) * 4 + 2 * ((k >> 4) & 1) + ((k >> 6) & 1)
    tot = np.zeros(v.shape[0])
    for gi in np.unique(grp):
        tot += w[:, grp == gi].max(axis=1)
    return (2.0 ** -10 * (1 + 2.0 ** -4) * tot)[:, None]


@pytest.mark.parametrize("dout,din,r,batch", [(d, n, r, b) for b in (1, 4, 16, 128) for d, n, r in SHAPES]
                         + [(256, 512, 128, 1024), (300, 200, 37, 1031)])
def test_config_distribution_stage_bounds(ctx, orc, dout, din, r, batch):
    say("factor stage bounds", dout, din, r, "batch", batch)
    rng = np.random.default_rng(1000 + dout + r + batch)
    L = make_layer(orc, rng, dout, din, r)
    layer = upload(ctx, L)
    x = orc.f32_to_bf16_fast(rng.standard_normal((batch, din)).astype(np.float32))
    y, ws = run_dev(layer, x)
    y2, _ = run_dev(layer, x)
    same(y, y2, "device result not repeatable")
    t = gpu_t(layer, ws, batch)
    tf = orc.bf16_to_f32(t).astype(np.float64)
    z = orc.bf16_to_f32(orc.f32_to_bf16_fast(L["s2"] * orc.bf16_to_f32(x))).astype(np.float64)
    t_exact = z @ L["vts"].T.astype(np.float64)
    assert np.all(np.abs(tf - t_exact) <= 1e-2 * np.abs(z).sum(axis=1, keepdims=True))
    _, t_orc = orc.factor_apply_bf16_batch(dout, din, r, L["ub"], L["vt"], L["s1"], L["s2"],
                                           L["bias"], x, want_t=True)
    tof = orc.bf16_to_f32(t_orc).astype(np.float64)
    ulp = np.spacing(np.abs(tof).astype(np.float32)).astype(np.float64) * 2 ** 16
    assert np.all(np.abs(tf - tof) <= ulp + 1e-6 * np.abs(z).sum(axis=1, keepdims=True) + mfma_window(z))
    # stage 2 from the device's own t
    u_exact = tf @ L["ubs"].T.astype(np.float64)
    y_exact = u_exact * L["s1"] + L["bias"]
    bound = np.abs(L["s1"]) * (1e-2 * np.abs(tf).sum(axis=1, keepdims=True)) + 1e-5 * np.abs(y_exact)
    assert np.all(np.abs(y - y_exact) <= bound)
    u_or = np.stack([orc.bf16_to_f32(orc.packed_matvec(L["ub"], dout, r, t[i], "bfloat16")) for i in range(batch)])
    y_or = (u_or * L["s1"] + L["bias"]).astype(np.float32)
    # one bf16 ulp of u, plus the f32 reassociation term (the device sums in a
    # different order; under cancellation that can move u across several ulps)
    # and the MFMA's summation window
    uulp = np.spacing(np.abs(u_or).astype(np.float32)) * 2 ** 16
    reassoc = 1e-6 * np.abs(tf).sum(axis=1, keepdims=True) + mfma_window(tf)
    assert np.all(np.abs(y - y_or) <= np.abs(L["s1"]) * (uulp * 1.01 + reassoc) + 1e-6 * np.abs(y_or))


def _rounding_layer(orc, rng, din, r=32):
    L = make_layer(orc, rng, 64, din, r)
    # scales that put a tie bit into the product's mantissa, overflow and underflow it
    picks = np.array([1 + 2.0 ** -8, 1.5 + 2.0 ** -9, 3.0, 2.0 ** 100, 2.0 ** -100, 1.0], np.float32)
    L["s2"] = np.where(rng.random(din) < 0.5, picks[rng.integers(0, picks.size, din)], L["s2"]).astype(np.float32)
    return L


def test_prefill_activation_rounding_staged(ctx, orc):
    """z = bf16(s2 * x) (engine/mod.rs:449-452), the two-stage prefill GEMM's
    first product (ranks past 2048 take that GEMM), for rows that are not
    16-byte chunks (din 203): staged whole at the head of the workspace and
    compared bit for bit with the oracle's rounding over ties, overflow to
    infinity, denormals and NaN payloads."""
    rng = np.random.default_rng(210)
    batch, din = 40, 203  # past the decode GEMV's 32 tokens, below the one-launch GEMM's 256
    L = _rounding_layer(orc, rng, din, r=2100)
    xb = rng.integers(0, 1 << 16, (batch, din)).astype(np.uint16)
    # every bf16 bit pattern class: NaNs with payloads, +-inf, denormals, zeros
    specials = np.array([0x7F81, 0x7FC0, 0xFFA5, 0x7F80, 0xFF80, 0x0001, 0x807F, 0x0000, 0x8000, 0x7F7F],
                        np.uint16)
    xb.ravel()[rng.choice(xb.size, 400, replace=False)] = specials[rng.integers(0, specials.size, 400)]
    layer = upload(ctx, L)
    _, ws = run_dev(layer, xb)
    din_p = -(-din // 64) * 64
    z = ws[: batch * din_p * 2].view(np.uint16).reshape(batch, din_p)
    want = orc.f32_to_bf16((L["s2"][None, :] * orc.bf16_to_f32(xb)).astype(np.float32))
    assert not z[:, din:].any()
    assert np.array_equal(z[:, :din], want), np.argwhere(z[:, :din] != want)[:5]


def _one_hot(orc, rng, L, batch, din, finite, zmax=np.inf):
    """x with one nonzero element per token, so that every sum of the two
    stages is exact: t = +-z of that element, u = (integer) * z.  Values are
    kept where z is a nonzero normal below zmax (or +-inf unless finite): the
    MFMA's NaN sign and denormal inputs are not IEEE-specified."""
    cols = rng.integers(0, din, batch)
    vals = np.zeros(batch, np.float32)
    for n in range(batch):
        while True:
            v = np.float32(rng.choice([-1, 1]) * 2.0 ** rng.uniform(-60, 60) * rng.uniform(1, 2))
            if not finite and rng.random() < 0.2:
                v = np.float32(rng.choice([-1, 1]) * 3.0e38)
            zf = orc.bf16_to_f32(orc.f32_to_bf16(np.float32(L["s2"][cols[n]] * orc.bf16_to_f32(orc.f32_to_bf16(v)))))
            if (np.isinf(zf) and not finite) or (np.isfinite(zf) and 2.0 ** -126 <= abs(zf) < zmax):
                vals[n] = v
                break
    x = np.zeros((batch, din), np.float32)
    x[np.arange(batch), cols] = vals
    return x, cols


def test_prefill_activation_rounding_fused(ctx, orc):
    """The same product formed inside the two-stage GEMM's activation staging
    (din % 8 == 0, rank past 2048): bf16 x through the device entry point,
    where t read back from the workspace must be exactly +-z, ties and
    overflow included; f32 x through the host face, where y must be
    bit-identical to the oracle's."""
    rng = np.random.default_rng(200)
    batch, din = 40, 200  # past the decode GEMV's 32 tokens, below the one-launch GEMM's 256
    L = _rounding_layer(orc, rng, din, r=2100)
    layer = upload(ctx, L)
    x, cols = _one_hot(orc, rng, L, batch, din, finite=False)
    xb = orc.f32_to_bf16(x)
    _, ws = run_dev(layer, xb)
    t = gpu_t(layer, ws, batch)
    z = orc.f32_to_bf16((L["s2"][cols] * orc.bf16_to_f32(xb[np.arange(batch), cols])).astype(np.float32))
    want = z[:, None] ^ np.where(L["vts"][:, cols].T < 0, np.uint16(0x8000), np.uint16(0))
    assert np.array_equal(t, want.astype(np.uint16)), np.argwhere(t != want)[:5]
    # f32 x (the host face uploads it aligned): staged as f32, y exact
    x, _ = _one_hot(orc, rng, L, batch, din, finite=True)
    got = layer.apply(x, "bfloat16")
    want_y = np.stack([orc.factor_apply("bf16", L["dout"], din, L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                        L["bias"], x[i]) for i in range(batch)])
    same(got, want_y)


@pytest.mark.parametrize("din", [200, 203])
def test_prefill_activation_rounding_one_launch(ctx, orc, din):
    """z = bf16(s2 * x) formed by the one-launch GEMM (gemm.hip) as it
    stages x: rows of 16-byte pieces (din 200) and element by element (din
    203).  One-hot tokens make every sum exact: t read back from the
    workspace must be exactly +-z over the tie-making scales, and y through
    the f32 host face bit-identical to the oracle's.  A token with an
    infinite z (s2 * x overflowing) gives NaN in every output where the
    reference's sequential composite does: its fp8 split turns inf into NaN,
    where the reference's t keeps +-inf and its u sums infinities of both
    signs.  The fp4 signs enter the MFMA as +-1.5 (divided out at the end),
    so sums whose 1.5-fold passes the f32 range overflow where the
    reference's stay finite: finite z are kept below 2^122 here (u sums r =
    32 of them)."""
    say("factor one-launch GEMM activation rounding", din)
    rng = np.random.default_rng(200 + din)
    batch = 1029  # the one-launch GEMM (from 256 tokens on); a ragged last group of 8
    L = _rounding_layer(orc, rng, din)
    layer = upload(ctx, L)
    zmax = 2.0 ** 122
    x, cols = _one_hot(orc, rng, L, batch, din, finite=True, zmax=zmax)
    xb = orc.f32_to_bf16(x)
    _, ws = run_dev(layer, xb)
    t = gpu_t(layer, ws, batch)
    z = orc.f32_to_bf16((L["s2"][cols] * orc.bf16_to_f32(xb[np.arange(batch), cols])).astype(np.float32))
    want = z[:, None] ^ np.where(L["vts"][:, cols].T < 0, np.uint16(0x8000), np.uint16(0))
    assert np.array_equal(t, want.astype(np.uint16)), np.argwhere(t != want)[:5]
    x, _ = _one_hot(orc, rng, L, batch, din, finite=True, zmax=zmax)
    got = layer.apply(x, "bfloat16")
    want_y = np.stack([orc.factor_apply("bf16", L["dout"], din, L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                                        L["bias"], x[i]) for i in range(batch)])
    same(got, want_y)
    x, _ = _one_hot(orc, rng, L, batch, din, finite=False, zmax=zmax)
    xb = orc.f32_to_bf16(x)
    want = orc.factor_apply_bf16_batch(L["dout"], din, L["r"], L["ub"], L["vt"], L["s1"], L["s2"], L["bias"], xb)
    got, _ = run_dev(layer, xb)
    assert np.isnan(want).any()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    same(got[fin], want[fin], "finite outputs")


def set_decode(S, x, dout):
    xd = torch.from_numpy(x.view(np.int16)).cuda()
    yd = torch.empty((x.shape[0], dout), dtype=torch.int16, device="cuda")
    ws = torch.zeros(S.workspace_size(), dtype=torch.uint8, device="cuda")
    S.decode_dev(xd, yd, ws, ws.numel(), torch.cuda.current_stream())
    torch.cuda.synchronize()
    return yd.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("dout,din,r,n", [(512, 1024, 200, 5), (300, 640, 200, 7), (96, 128, 64, 3)])
def test_set_decode_matches_single_layers(ctx, orc, dout, din, r, n, f16):
    """Integer-exact set decode: bit-identical to the oracle and to the
    single-layer path (steps of fewer than 8 slices where din/128 or r_p/128
    is small).  With s1, s2 and bias fp16 values (f16, as a v2 qpk1 stream
    holds them) the decode streams the layers' fp16 copies: s2 in the
    operand prep, s1 and bias in stage 2's epilogue."""
    from quantibbler_amd import FactorSet

    say("factor set decode", dout, din, r, n, "fp16 scales" if f16 else "")
    rng = np.random.default_rng(77 + din)
    Ls = [make_layer(orc, rng, dout, din, r, integer=True) for _ in range(n)]
    if f16:
        for L in Ls:
            for k in ("s1", "s2", "bias"):
                L[k] = L[k].astype(np.float16).astype(np.float32)
    layers = [upload(ctx, L) for L in Ls]
    S = FactorSet(ctx, layers)
    x = orc.f32_to_bf16_fast(rng.integers(-2, 3, (n, din)).astype(np.float32))
    ys = set_decode(S, x, dout)
    for i, (L, layer) in enumerate(zip(Ls, layers)):
        want = orc.factor_apply_bf16_batch(dout, din, r, L["ub"], L["vt"], L["s1"], L["s2"], L["bias"],
                                           x[i:i + 1])
        wb = orc.f32_to_bf16_fast(want)[0]
        same(ys[i], wb, f"set decode, layer {i}")
        yi, _ = run_dev(layer, x[i:i + 1], "bfloat16")
        same(ys[i], yi[0])


def test_decode_flat_prep_matches_layer_prep(ctx, orc):
    """At batch 1 with every din a multiple of 128 and x 16-byte aligned,
    stage 1's fp8 operand comes from the flat prep (run t of the whole x, no
    per-layer lookup); with x misaligned, from the per-layer prep.  Same
    layer, same x values (real-valued, so every rounding matters): the two
    outputs are bit-identical."""
    say("factor decode flat prep vs per-layer prep")
    rng = np.random.default_rng(123)
    for dout, din, r in [(1024, 4096, 1102), (640, 1024, 200)]:
        L = make_layer(orc, rng, dout, din, r)
        layer = upload(ctx, L)
        x = orc.f32_to_bf16_fast((3.0 * rng.standard_normal(din)).astype(np.float32))
        xa = torch.from_numpy(x.view(np.int16)).cuda()                     # aligned: flat prep
        xm = torch.empty(din + 1, dtype=torch.int16, device="cuda")[1:]    # 2 bytes off: layer prep
        xm.copy_(xa)
        assert xa.data_ptr() % 16 == 0 and xm.data_ptr() % 16 != 0
        outs = []
        for xd in (xa, xm):
            y = torch.empty(dout, dtype=torch.int16, device="cuda")
            ws = torch.zeros(layer.workspace_size(1), dtype=torch.uint8, device="cuda")
            layer.linear_dev(xd, 1, y, "bfloat16", ws, ws.numel(), torch.cuda.current_stream())
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy().view(np.uint16))
        assert np.all(np.isfinite(orc.bf16_to_f32(outs[0])))
        assert np.array_equal(outs[0], outs[1]), np.argwhere(outs[0] != outs[1])[:5]


def test_mixed_shape_set_decode(ctx, orc):
    """One set over layers of different shapes (a decoder layer's q/k/v/o/
    gate/up/down, scaled down, with ragged ranks and a din that is not a
    multiple of 8): x and y are the concatenated per-layer vectors, every
    layer's output bit-identical to the oracle on integer-exact inputs."""
    from quantibbler_amd import FactorSet

    say("factor mixed-shape set decode")
    rng = np.random.default_rng(91)
    shapes = [(512, 512, 138), (128, 512, 54), (128, 512, 54), (512, 512, 138), (1792, 512, 216),
              (1792, 512, 216), (512, 1792, 217), (200, 300, 37)]
    Ls = [make_layer(orc, rng, m, n, r, integer=True) for m, n, r in shapes]
    layers = [upload(ctx, L) for L in Ls]
    S = FactorSet(ctx, layers)
    xs = [orc.f32_to_bf16_fast(rng.integers(-2, 3, n).astype(np.float32)) for _, n, _ in shapes]
    x = np.concatenate(xs)
    xd = torch.from_numpy(x.view(np.int16)).cuda()
    yd = torch.empty(sum(m for m, _, _ in shapes), dtype=torch.int16, device="cuda")
    ws = torch.zeros(S.workspace_size(), dtype=torch.uint8, device="cuda")
    for rep in range(2):  # the workspace keeps the last call's contents: run twice
        S.decode_dev(xd, yd, ws, ws.numel(), torch.cuda.current_stream())
        torch.cuda.synchronize()
        y = yd.cpu().numpy().view(np.uint16)
        off = 0
        for i, ((m, n, r), L, xi) in enumerate(zip(shapes, Ls, xs)):
            want = orc.factor_apply_bf16_batch(m, n, r, L["ub"], L["vt"], L["s1"], L["s2"], L["bias"],
                                               xi[None, :])
            same(y[off:off + m], orc.f32_to_bf16_fast(want)[0], f"mixed set, layer {i} {(m, n, r)}")
            off += m


def test_apply_host_faces(ctx, orc):
    say("factor apply host faces")
    rng = np.random.default_rng(5)
    L = make_layer(orc, rng, 96, 160, 40)
    layer = upload(ctx, L)
    x = rng.standard_normal(160).astype(np.float32)
    # fp32 serving: f64 matvecs in element order -> bit-identical (BS-3.1)
    got = layer.apply(x, "float32")
    want = orc.factor_apply("fp32", 96, 160, 40, L["ub"], L["vt"], L["s1"], L["s2"], L["bias"], x)
    same(got, want)
    xs = rng.standard_normal((3, 160)).astype(np.float32)
    got3 = layer.apply(xs, "float32")
    for i in range(3):
        same(got3[i], orc.factor_apply("fp32", 96, 160, 40, L["ub"], L["vt"], L["s1"], L["s2"], L["bias"], xs[i]))
    # bf16 serving with an f32 x: z = bf16(s2*x) as apply_bf16 does
    got_b = layer.apply(x, "bfloat16")
    want_b = orc.factor_apply("bf16", 96, 160, 40, L["ub"], L["vt"], L["s1"], L["s2"], L["bias"], x)
    z = orc.bf16_to_f32(orc.f32_to_bf16_fast(L["s2"] * x)).astype(np.float64)
    tf = np.abs(z).sum() * 2  # loose scale for the two-stage bound
    assert np.all(np.abs(got_b - want_b) <= np.abs(L["s1"]) * 1e-2 * tf)


def qpk1_stream(L, orc):
    dout, din, r = L["dout"], L["din"], L["r"]
    ub_bits = np.zeros((dout * r + 7) // 8, np.uint8)
    vb_bits = np.zeros((din * r + 7) // 8, np.uint8)
    for i in range(dout):
        for j in range(r):
            if L["ubs"][i, j] == 1:
                b = i * r + j
                ub_bits[b >> 3] |= 1 << (b & 7)
    vb = L["vts"].T  # (din, r)
    for i in range(din):
        for j in range(r):
            if vb[i, j] == 1:
                b = i * r + j
                vb_bits[b >> 3] |= 1 << (b & 7)
    head = b"QPK1" + b"".join(int(v).to_bytes(4, "little") for v in (2, 1, dout, din, r))
    f16 = lambda a: np.asarray(a, np.float16).tobytes()
    return head + f16(L["s1"]) + f16(L["s2"]) + f16(L["bias"]) + ub_bits.tobytes() + vb_bits.tobytes()


def test_from_qpk1_matches_from_rows(ctx, orc):
    from quantibbler_amd import FactorLayer, KernelError

    say("factor from qpk1")
    rng = np.random.default_rng(6)
    L = make_layer(orc, rng, 40, 24, 13)
    L["s1"] = L["s1"].astype(np.float16).astype(np.float32)
    L["s2"] = L["s2"].astype(np.float16).astype(np.float32)
    L["bias"] = L["bias"].astype(np.float16).astype(np.float32)
    stream = qpk1_stream(L, orc)
    parsed = orc.qpk1_parse(stream)
    assert np.array_equal(orc.container_to_rows(parsed["ub_packed"], 40, 13), L["ub"].ravel())
    assert np.array_equal(orc.container_to_rows_transposed(parsed["vb_packed"], 24, 13), L["vt"].ravel())
    a = FactorLayer.from_qpk1(ctx, stream)
    b = upload(ctx, L)
    x = orc.f32_to_bf16_fast(rng.standard_normal((3, 24)).astype(np.float32))
    same(run_dev(a, x)[0], run_dev(b, x)[0])
    with pytest.raises(KernelError, match="trailing garbage"):
        FactorLayer.from_qpk1(ctx, stream + b"\0")


def gpu_z(layer, ws, batch):
    """Stage 1's fp8 operand read back from the decode workspace
    ([op1 [slice][4][ncol][32] | sc1 [slice][4][ncol] | ...]): the value
    hi + lo each activation z = bf16(s2*x) is fed to the MFMA as."""
    rnd = lambda n: -(-n // 256) * 256
    ns1, ncol = -(-layer.din // 128), 2 * batch
    op = ws[: ns1 * 4 * ncol * 32].reshape(ns1, 4, ncol, 32)
    sc = ws[rnd(ns1 * 4 * ncol * 32):][: ns1 * 4 * ncol].reshape(ns1, 4, ncol).astype(np.int64)
    z = np.zeros((batch, ns1 * 128))
    for g in range(4):
        for e in range(32):
            gb, byte, k = 2 * (g & 1) + (e >> 4), 16 * (g >> 1) + (e & 15), kq4(g, e)
            for b in range(batch):
                hi = e4m3(op[:, gb, 2 * b, byte]) * 2.0 ** (sc[:, g, 2 * b] - 127)
                lo = e4m3(op[:, gb, 2 * b + 1, byte]) * 2.0 ** (sc[:, g, 2 * b + 1] - 127)
                z[b, np.arange(ns1) * 128 + k] = hi + lo
    return z[:, :layer.din]


def test_decode_fp8_split_tail(ctx, orc):
    """The decode GEMV feeds each activation z to the fp4 x fp8 MFMA as two
    e4m3 pieces, hi + lo, each scaled by one E8M0 exponent per 32-activation
    group (the two 16-runs MFMA lane group g covers).  Every z within 2^14
    of its group's largest |z| is carried exactly; smaller ones can lose low
    bits in the e4m3 subnormals, by at most 2^-21 of the group maximum (the
    lo piece's subnormal step is 2^-9 of its scale, which is at most 2^-7 of
    the largest residual, itself at most 2^-4 of the group maximum).  Groups
    built here: one element 2^10, the others 2^-8 .. 2^2 with full 8-bit
    mantissas, some zero."""
    say("factor decode fp8 split tail")
    rng = np.random.default_rng(4321)
    din = 256
    L = make_layer(orc, rng, 64, din, 64, integer=True)
    layer = upload(ctx, L)
    batch = 2
    mags = 2.0 ** rng.integers(-8, 3, (batch, din)) * (1 + rng.integers(0, 128, (batch, din)) / 128.0)
    x = (rng.choice([-1, 1], (batch, din)) * mags).astype(np.float32)
    x[rng.random((batch, din)) < 0.05] = 0.0
    groups = [np.concatenate([np.arange(16) + 16 * (g >> 1) + 64 * (g & 1),
                              np.arange(16) + 16 * (g >> 1) + 64 * (g & 1) + 32]) for g in range(4)]
    for b in range(batch):
        for s in range(din // 128):
            for g in range(4):
                x[b, 128 * s + rng.choice(groups[g])] = rng.choice([-1, 1]) * 1024.0
    xb = orc.f32_to_bf16_fast(x)
    _, ws = run_dev(layer, xb)
    zd = gpu_z(layer, ws, batch)
    z = orc.bf16_to_f32(xb).astype(np.float64)
    inexact = 0
    for b in range(batch):
        for s in range(din // 128):
            for g in range(4):
                k = 128 * s + groups[g]
                amax = np.abs(z[b, k]).max()
                err = np.abs(zd[b, k] - z[b, k])
                near = np.abs(z[b, k]) >= amax * 2.0 ** -14
                assert not err[near].any(), (b, s, g)
                assert np.all(err <= amax * 2.0 ** -21), (b, s, g, err.max() / amax)
                inexact += int((err > 0).sum())
    say(f"  {inexact} of {z.size} activations below 2^-14 of their group maximum lost low bits")


def test_decode_nonfinite_activations(ctx, orc):
    """inf, NaN and overflow of s2*x to inf on the decode path (batch 4, one
    clean token): the clean token stays bit-identical to the oracle; a token
    holding a non-finite z gives NaN in every output where the reference's
    sequential composite does (with random signs and r >= 2 every u sums
    infinities of both signs), and the same finite values elsewhere."""
    say("factor decode non-finite activations")
    rng = np.random.default_rng(4322)
    din, r, dout = 256, 64, 96
    L = make_layer(orc, rng, dout, din, r, integer=True)
    L["s2"][7] = np.float32(2.0 ** 120)
    layer = upload(ctx, L)
    x = rng.integers(-2, 3, (4, din)).astype(np.float32)
    x[:, 7] = 0.0
    x[0, 3] = np.inf
    x[2, 7] = 1024.0          # s2 * x = 2^130: inf in f32 and bf16
    x[3, 100] = np.nan
    xb = orc.f32_to_bf16_fast(x)
    xb[1, 7] = 0x3F80          # the clean token: z_7 = 2^120, a finite term that swamps the rest
    want = orc.factor_apply_bf16_batch(dout, din, r, L["ub"], L["vt"], L["s1"], L["s2"], L["bias"], xb)
    got, _ = run_dev(layer, xb)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    same(got[fin], want[fin], "finite outputs")
    assert np.isnan(want[[0, 2, 3]]).all() and np.isfinite(want[1]).all()
