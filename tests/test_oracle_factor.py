"""Pin the oracle's factor-linear composite and the qpk1 reader.

Known answers: the engine's hand-derived 4x4 r=8 layer and bias tests
(crates/quantibbler-server/src/engine/mod.rs:1533-1664), the container ->
row repack KAT (:1583-1600), the fp32 byte-identity construction
(:1865-1891), the bf16 stage bound (:1897-1949), and the qpk1 hex KATs
(crates/quantibbler-qpk1/src/lib.rs:334-410).
"""
import numpy as np
import pytest


def layer_fixture(orc):
    dout, din, r = 4, 4, 8
    ub_signs = np.array([
        1, -1, 1, 1, -1, 1, -1, -1,
        1, 1, 1, -1, -1, -1, 1, 1,
        -1, 1, -1, -1, 1, -1, 1, 1,
        1, -1, -1, 1, 1, 1, -1, -1], np.int8)
    ub = np.zeros(dout * r // 8, np.uint8)
    for idx, s in enumerate(ub_signs):
        if s == 1:
            ub[idx >> 3] |= 1 << (idx & 7)
    vb = np.full(din * r // 8, 0xFF, np.uint8)
    s1 = np.array([1.0, 0.5, -2.0, 0.25], np.float32)
    s2 = np.array([0.25, -0.5, 2.0, 1.0], np.float32)
    return dout, din, r, ub, vb, s1, s2, ub_signs.reshape(dout, r)


def test_container_to_rows_kat(orc):
    signs = [[1, -1, 1, -1, 1], [-1, -1, 1, 1, -1]]
    container = np.zeros(2, np.uint8)
    for i, row in enumerate(signs):
        for j, s in enumerate(row):
            if s == 1:
                container[(i * 5 + j) >> 3] |= 1 << ((i * 5 + j) & 7)
    rows = orc.container_to_rows(container, 2, 5)
    assert rows.tolist() == [0b0001_0101, 0b0000_1100]


def test_layer_apply_matches_dense(orc):
    dout, din, r, ub, vb, s1, s2, ubs = layer_fixture(orc)
    ub_rows = orc.container_to_rows(ub, dout, r)
    vbt = orc.container_to_rows_transposed(vb, din, r)
    assert ub_rows.tolist() == ub.tolist()  # r % 8 == 0: layouts coincide
    x = np.array([0.5, -1.25, 2.0, 0.0], np.float32)
    z = s2.astype(np.float64) * x
    vt_z = z.sum()
    expected = np.array([s1[i] * sum(ubs[i, k] * vt_z for k in range(r)) for i in range(dout)])
    got = orc.factor_apply("fp32", dout, din, r, ub_rows, vbt, s1, s2, None, x)
    assert np.all(np.abs(got - expected) < 1e-4)
    # bias is added per output feature (engine/mod.rs:1637-1664)
    bias = np.array([0.5, -1.5, 2.0, -0.25], np.float32)
    got_b = orc.factor_apply("fp32", dout, din, r, ub_rows, vbt, s1, s2, bias, x)
    assert np.all(np.abs(got_b.astype(np.float64) - (got.astype(np.float64) + bias)) < 1e-6)


def test_fp32_path_byte_identity_construction(orc):
    # engine/mod.rs:1865-1891: f64 z, f64-accumulating kernel, f32 scale/bias
    rng = np.random.default_rng(3)
    dout, din, r = 33, 70, 19
    ub_rows = orc.pack_bits(rng.choice([-1, 1], (dout, r)).astype(np.int8))
    vbt = orc.pack_bits(rng.choice([-1, 1], (r, din)).astype(np.int8))
    s1 = np.exp(0.5 * rng.standard_normal(dout)).astype(np.float32)
    s2 = np.exp(0.5 * rng.standard_normal(din)).astype(np.float32)
    b = rng.standard_normal(dout).astype(np.float32)
    x = rng.standard_normal(din).astype(np.float32)
    z = (s2 * x).astype(np.float64)
    t = orc.packed_matvec(vbt, r, din, z)
    u = orc.packed_matvec(ub_rows, dout, r, t)
    want = (u.astype(np.float32) * s1 + b).astype(np.float32)
    got = orc.factor_apply("fp32", dout, din, r, ub_rows, vbt, s1, s2, b, x)
    assert got.tobytes() == want.tobytes()
    fast = orc.factor_apply("fp32", dout, din, r, ub_rows, vbt, s1, s2, b, x, fast=True)
    assert np.all(np.abs(fast - got) <= 1e-5 * np.abs(got).max())


def test_bf16_composite_stage_bound_and_batch_form(orc):
    # engine/mod.rs:1897-1949: bf16 stage within 1e-2 of the row term scale
    rng = np.random.default_rng(4)
    dout, din, r = 40, 96, 24
    ubs = rng.choice([-1, 1], (dout, r)).astype(np.int8)
    vts = rng.choice([-1, 1], (r, din)).astype(np.int8)
    ub_rows, vbt = orc.pack_bits(ubs), orc.pack_bits(vts)
    s1 = np.exp(0.5 * rng.standard_normal(dout)).astype(np.float32)
    s2 = np.exp(0.5 * rng.standard_normal(din)).astype(np.float32)
    x = rng.standard_normal(din).astype(np.float32)
    z = orc.bf16_to_f32(orc.f32_to_bf16(s2 * x)).astype(np.float64)
    t_exact = vts.astype(np.float64) @ z
    y = orc.factor_apply("bf16", dout, din, r, ub_rows, vbt, s1, s2, None, x)
    # rebuild t the way apply_bf16 does and bound it against the exact product
    t = orc.packed_matvec(vbt, r, din, orc.f32_to_bf16(s2 * x), "bfloat16")
    assert np.all(np.abs(orc.bf16_to_f32(t) - t_exact) <= 1e-2 * np.abs(z).sum())
    u = orc.packed_matvec(ub_rows, dout, r, t, "bfloat16")
    assert y.tobytes() == (orc.bf16_to_f32(u) * s1).astype(np.float32).tobytes()
    # the batched token-major form equals the per-token form when x is bf16
    xb = orc.f32_to_bf16(rng.standard_normal((3, din)).astype(np.float32))
    yb, tb = orc.factor_apply_bf16_batch(dout, din, r, ub_rows, vbt, s1, s2, None, xb, want_t=True)
    for i in range(3):
        yi = orc.factor_apply("bf16", dout, din, r, ub_rows, vbt, s1, s2, None, orc.bf16_to_f32(xb[i]))
        assert yb[i].tobytes() == yi.tobytes()


V1 = bytes.fromhex("51504b31" "01000000" "01000000" "03000000" "05000000" "07000000"
                   "003c003800c0" "003400b80040003c0030" "2b7307" "55e6413503")
V2 = bytes.fromhex("51504b31" "02000000" "01000000" "03000000" "05000000" "03000000"
                   "003c003800c0" "003400b80040003c0030" "003c00b80040" "7301" "e535")


def test_qpk1_v1_kat(orc):
    L = orc.qpk1_parse(V1)
    assert (L["version"], L["dout"], L["din"], L["r"], L["dtype_tag"]) == (1, 3, 5, 7, 1)
    assert L["s1"].tolist() == [1.0, 0.5, -2.0]
    assert L["s2"].tolist() == [0.25, -0.5, 2.0, 1.0, 0.125]
    assert L["bias"].size == 0
    assert L["ub_packed"].tolist() == [0x2B, 0x73, 0x07]
    assert L["vb_packed"].tolist() == [0x55, 0xE6, 0x41, 0x35, 0x03]


def test_qpk1_v2_kat_and_rejections(orc):
    assert len(V2) == 50 == orc.qpk1_expected_size(3, 5, 3, 2, True)
    L = orc.qpk1_parse(V2)
    assert L["version"] == 2 and L["bias"].tolist() == [1.0, -0.5, 2.0]
    assert L["ub_packed"].tolist() == [0x73, 0x01] and L["vb_packed"].tolist() == [0xE5, 0x35]
    legacy = bytearray(V2)
    del legacy[40:46]
    legacy[4:8] = (1).to_bytes(4, "little")
    L1 = orc.qpk1_parse(bytes(legacy))
    assert L1["version"] == 1 and L1["ub_packed"].tolist() == [0x73, 0x01]
    with pytest.raises(orc.OracleError, match="truncated stream: 49 bytes; header declares 50"):
        orc.qpk1_parse(V2[:-1])
    with pytest.raises(orc.OracleError, match="trailing garbage: 51 bytes; one layer at this header is 50"):
        orc.qpk1_parse(V2 + b"\0")
    with pytest.raises(orc.OracleError, match="bad magic"):
        orc.qpk1_parse(b"QPK2" + V2[4:])
    with pytest.raises(orc.OracleError, match="unsupported representation version 3"):
        orc.qpk1_parse(V2[:4] + (3).to_bytes(4, "little") + V2[8:])
    with pytest.raises(orc.OracleError, match="unknown dtype tag 7"):
        orc.qpk1_parse(V2[:8] + (7).to_bytes(4, "little") + V2[12:])
    with pytest.raises(orc.OracleError, match="shorter than the 24-byte header"):
        orc.qpk1_parse(V2[:10])
