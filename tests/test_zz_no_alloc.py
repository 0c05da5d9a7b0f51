"""The no-allocation factor linear (qbk_factor_linear_noalloc_dev) against
qbk_factor_linear_dev on the same layer and inputs: bit-identical outputs on
two calls in a row, the second with a smaller input (its scratch array keeps
the first call's contents), for the decode GEMV (batch <= 32) and the prefill
GEMM; the call captured in a HIP graph and replayed with new inputs; and
the refusal of a call whose workspace exceeds the array."""
import numpy as np
import pytest

from conftest import same

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    from quantibbler_amd import GpuContext

    return GpuContext(0)


def _layer(ctx, orc, rng, dout, din, r):
    from quantibbler_amd import FactorLayer

    ubs = rng.choice([-1, 1], (dout, r)).astype(np.int8)
    vts = rng.choice([-1, 1], (r, din)).astype(np.int8)
    return FactorLayer.from_rows(ctx, dout, din, r, orc.pack_bits(ubs), orc.pack_bits(vts),
                                 np.exp(0.5 * rng.standard_normal(dout)).astype(np.float32),
                                 np.exp(0.5 * rng.standard_normal(din)).astype(np.float32),
                                 rng.standard_normal(dout).astype(np.float32))


def _with_workspace(layer, x, y_dtype):
    batch = x.shape[0]
    y = torch.empty((batch, layer.dout), dtype=torch.float32 if y_dtype == "float32" else torch.int16,
                    device="cuda")
    n = layer.workspace_size(batch)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    layer.linear_dev(x, batch, y, y_dtype, ws, n, torch.cuda.current_stream())
    return y


def _no_alloc(layer, x, y_dtype):
    batch = x.shape[0]
    y = torch.empty((batch, layer.dout), dtype=torch.float32 if y_dtype == "float32" else torch.int16,
                    device="cuda")
    layer.linear_noalloc_dev(x, batch, y, y_dtype, torch.cuda.current_stream())
    return y


@pytest.mark.parametrize("dout,din,r,first,second", [(1024, 4096, 1102, 8, 1), (512, 1024, 200, 300, 17),
                                                     (300, 200, 37, 5, 2)])
def test_no_alloc_matches_workspace_form(ctx, orc, dout, din, r, first, second):
    say("no-alloc factor linear", dout, din, r, first, second)
    rng = np.random.default_rng(dout + first)
    layer = _layer(ctx, orc, rng, dout, din, r)
    for batch in (first, second):
        xb = orc.f32_to_bf16_fast(rng.standard_normal((batch, din)).astype(np.float32))
        x = torch.from_numpy(xb.view(np.int16)).cuda()
        for y_dtype in ("float32", "bfloat16"):
            want = _with_workspace(layer, x, y_dtype)
            got = _no_alloc(layer, x, y_dtype)
            torch.cuda.synchronize()
            same(got.cpu().numpy(), want.cpu().numpy(), f"batch {batch} {y_dtype}")
    layer.close()


def test_no_alloc_refuses_beyond_its_array(ctx, orc):
    from quantibbler_amd import KernelError

    say("no-alloc factor linear: size limit")
    rng = np.random.default_rng(9)
    layer = _layer(ctx, orc, rng, 4096, 4096, 1024)
    batch = 2048
    while layer.workspace_size(batch) <= 32 << 20:
        batch *= 2
    x = torch.zeros((batch, 4096), dtype=torch.int16, device="cuda")
    y = torch.empty((batch, 4096), dtype=torch.float32, device="cuda")
    with pytest.raises(KernelError, match="the no-allocation entry point holds 33554432"):
        layer.linear_noalloc_dev(x, batch, y, "float32", torch.cuda.current_stream())
    layer.close()


@pytest.mark.parametrize("dout,din,r,batch", [(1024, 4096, 1102, 1), (512, 1024, 200, 300)])
def test_no_alloc_under_graph_capture(ctx, orc, dout, din, r, batch):
    """The no-allocation call captured in a HIP graph (torch's graph API) after
    one eager call on the device (the scratch address is looked up there),
    then replayed with new inputs written into the captured input buffer:
    every replay bit-identical to qbk_factor_linear_dev on the same input,
    with eager work and synchronisations between the replays."""
    say("no-alloc factor linear under graph capture", dout, din, r, batch)
    rng = np.random.default_rng(dout + batch + 1)
    layer = _layer(ctx, orc, rng, dout, din, r)
    x = torch.zeros((batch, din), dtype=torch.int16, device="cuda")
    y = torch.zeros((batch, dout), dtype=torch.float32, device="cuda")
    layer.linear_noalloc_dev(x, batch, y, "float32", torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer.linear_noalloc_dev(x, batch, y, "float32", torch.cuda.current_stream())
    for rep in range(3):
        xb = orc.f32_to_bf16_fast(rng.standard_normal((batch, din)).astype(np.float32))
        x.copy_(torch.from_numpy(xb.view(np.int16)))
        g.replay()
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        want = _with_workspace(layer, x, "float32")
        torch.cuda.synchronize()
        same(got, want.cpu().numpy(), f"replay {rep}")
    del g
    layer.close()
