"""GPU parity of the qpk1 layer loader (crates/quantibbler-qpk1/src/lib.rs:
229-320 parse, engine/mod.rs:342-381 PackedLayer::from_layer) through the
product parser qbk_factor_from_qpk1, on the reference's own data:

* the v1 48-byte and v2 50-byte hex KATs (lib.rs:334-410) and the v1
  sibling of the v2 stream;
* every layer file of the reference's fixture models (parity-tiny: 14
  layers, v1, f16; server-model, -bias (v2), -bf16: 7 layers each);
* the same layers re-serialised with the float32 scale tag (tag 2), which no
  reference file carries;
* the parse rejections, whose texts must equal the reference's.

Each uploaded layer is checked against the oracle's parse + composite:
the fp32-serving face (f64 sums in element order) bit-identical on random
x; the bf16-serving face bit-identical on one-hot x (one nonzero element
per token, so every sum of both stages is exact and every rounding is
decided by the exact value), at batch 1 and 5 (decode GEMV) and at batch din
(prefill GEMM, every column of Vb exercised).
"""
import glob
import os

import numpy as np
import pytest

from conftest import GOLDEN, same

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

V1 = bytes.fromhex("51504b31" "01000000" "01000000" "03000000" "05000000" "07000000"
                   "003c003800c0" "003400b80040003c0030" "2b7307" "55e6413503")
V2 = bytes.fromhex("51504b31" "02000000" "01000000" "03000000" "05000000" "03000000"
                   "003c003800c0" "003400b80040003c0030" "003c00b80040" "7301" "e535")


def _v1_sibling():
    b = bytearray(V2)
    del b[40:46]
    b[4:8] = (1).to_bytes(4, "little")
    return bytes(b)


def fixture_files():
    return sorted(glob.glob(os.path.join(GOLDEN, "*", "layers", "**", "*.qpk1"), recursive=True))


def as_f32_tag(stream, orc):
    """The same layer with float32 scales (dtype tag 2)."""
    L = orc.qpk1_parse(stream)
    head = stream[:8] + (2).to_bytes(4, "little") + stream[12:24]
    body = L["s1"].astype(np.float32).tobytes() + L["s2"].astype(np.float32).tobytes()
    if L["version"] >= 2:
        body += L["bias"].astype(np.float32).tobytes()
    return head + body + L["ub_packed"].tobytes() + L["vb_packed"].tobytes()


def streams(orc):
    out = [("kat_v1", V1), ("kat_v2", V2), ("kat_v2_v1_sibling", _v1_sibling())]
    for f in fixture_files():
        with open(f, "rb") as fh:
            out.append((os.path.relpath(f, GOLDEN), fh.read()))
    for name, s in list(out[:3]) + [o for o in out if "q_proj" in o[0] or "down_proj" in o[0]][:6]:
        out.append((name + "@f32", as_f32_tag(s, orc)))
    return out


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def one_hot(orc, rng, batch, din, cols=None):
    cols = rng.integers(0, din, batch) if cols is None else np.asarray(cols)
    x = np.zeros((batch, din), np.float32)
    x[np.arange(batch), cols] = (rng.choice([-1, 1], batch) * 2.0 ** rng.integers(-3, 4, batch)).astype(np.float32)
    return orc.f32_to_bf16_fast(x)


def test_fixture_inventory():
    files = fixture_files()
    assert len(files) == 35, len(files)


def test_qpk1_layers_through_the_product_parser(ctx, orc):
    from quantibbler_amd import FactorLayer

    rng = np.random.default_rng(1717)
    for name, s in streams(orc):
        print("qpk1", name, len(s), flush=True)
        L = orc.qpk1_layer(s)
        dev = FactorLayer.from_qpk1(ctx, s)
        assert (dev.dout, dev.din, dev.r) == (L["dout"], L["din"], L["r"]), name
        # fp32 serving: bit-identical on random x
        x = rng.standard_normal((2, L["din"])).astype(np.float32)
        got = dev.apply(x, "float32")
        for i in range(2):
            want = orc.factor_apply("fp32", L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"],
                                    L["s2"], L["bias"], x[i])
            same(got[i], want, f"{name}: fp32 face")
        # bf16 serving on one-hot x: decode (1, 5) and GEMM (every column)
        for xb in (one_hot(orc, rng, 1, L["din"]), one_hot(orc, rng, 5, L["din"]),
                   one_hot(orc, rng, max(L["din"], 9), L["din"], np.arange(max(L["din"], 9)) % L["din"])):
            batch = xb.shape[0]
            want = orc.factor_apply_bf16_batch(L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"],
                                               L["s2"], L["bias"], xb)
            xd = torch.from_numpy(xb.view(np.int16)).cuda()
            yd = torch.empty((batch, L["dout"]), dtype=torch.float32, device="cuda")
            wn = dev.workspace_size(batch)
            ws = torch.zeros(wn, dtype=torch.uint8, device="cuda")
            dev.linear_dev(xd, batch, yd, "float32", ws, wn, torch.cuda.current_stream())
            torch.cuda.synchronize()
            same(yd.cpu().numpy(), want, f"{name}: bf16 face, batch {batch}")
        dev.close()


def test_qpk1_rejections_carry_the_reference_texts(ctx, orc):
    from quantibbler_amd import FactorLayer, KernelError

    bad = [
        (V2[:10], "stream is 10 bytes; shorter than the 24-byte header"),
        (b"XPK1" + V2[4:], "bad magic [88, 80, 75, 49]; expected [81, 80, 75, 49]"),
        (V2[:4] + (7).to_bytes(4, "little") + V2[8:], "unsupported representation version 7; this reader "
         "implements version 1 (pre-bias legacy) and version 2 (current, with bias)"),
        (V2[:8] + (9).to_bytes(4, "little") + V2[12:], "unknown dtype tag 9; expected 1 (float16) or 2 (float32)"),
        (V2[:20] + (0).to_bytes(4, "little") + V2[24:], "dout, din and r must all be >= 1, got (3, 5, 0)"),
        (V2[:44], "truncated stream: 44 bytes; header declares 50"),
        (V2 + b"\0", "trailing garbage: 51 bytes; one layer at this header is 50"),
    ]
    for stream, text in bad:
        with pytest.raises(KernelError) as ei:
            FactorLayer.from_qpk1(ctx, stream)
        assert str(ei.value) == text
        with pytest.raises(orc.OracleError) as eo:
            orc.qpk1_parse(stream)
        assert str(eo.value) == text
