"""GPU parity: the language-model head (engine/mod.rs:781-800 Engine::logits)
through the C ABI -- bit-identical to the oracle's sequential f32 sums, for
bf16-valued heads (stored as bf16) and f32 heads (stored as f32), ragged
vocabularies, d_model not a multiple of the 64-step load chunks, batches of
1-70 rows (a launch takes up to 32, in 1, 2 or 4 wave chunks of up to 8 with
a shorter last chunk), and the device-pointer form."""
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


@pytest.mark.parametrize("vocab,d,bf16,batch", [
    (1000, 64, True, 1), (777, 100, True, 3), (1537, 256, False, 2), (513, 4096, True, 11), (300, 7, False, 8),
    # whole 128-step chunks and a ragged tail that ends inside a four-step group
    (650, 262, True, 2), (130, 262, False, 1),
    # two chunks (9-16 rows), four (17-32), and several launches
    (1000, 300, True, 9), (700, 128, False, 16), (1500, 200, True, 17), (513, 520, True, 32),
    (300, 100, False, 30), (1100, 96, True, 70),
])
def test_head_logits_bit_identical(ctx, orc, vocab, d, bf16, batch):
    from quantibbler_amd import LmHead

    say("lm_head", vocab, d, bf16, batch)
    rng = np.random.default_rng(vocab + d + batch)
    head = rng.standard_normal((vocab, d)).astype(np.float32)
    x = rng.standard_normal((batch, d)).astype(np.float32)
    if bf16:  # bf16 serving: both operands bf16 values
        head = orc.bf16_to_f32(orc.f32_to_bf16_fast(head))
        x = orc.bf16_to_f32(orc.f32_to_bf16_fast(x))
    H = LmHead.from_rows(ctx, head)
    assert H.bf16 == bf16 and H.vocab == vocab and H.d_model == d
    got = H.logits(x)
    want = orc.head_logits(head, x)
    same(got, want, "host form")
    xd = torch.from_numpy(x).cuda()
    out = torch.empty((batch, vocab), dtype=torch.float32, device="cuda")
    H.logits_dev(xd, batch, out, torch.cuda.current_stream())
    torch.cuda.synchronize()
    same(out.cpu().numpy(), want, "device form")
    H.close()


def test_head_from_device_rows_and_validation(ctx, orc):
    import ctypes as C

    from quantibbler_amd import KernelError, LmHead, _lib

    rng = np.random.default_rng(9)
    head = orc.bf16_to_f32(orc.f32_to_bf16_fast(rng.standard_normal((600, 96)).astype(np.float32)))
    H = LmHead.from_rows_dev(ctx, torch.from_numpy(head).cuda(), 600, 96)
    assert H.bf16
    x = orc.bf16_to_f32(orc.f32_to_bf16_fast(rng.standard_normal(96).astype(np.float32)))
    same(H.logits(x), orc.head_logits(head, x))
    with pytest.raises(KernelError, match="hidden must hold rows of d_model = 96 values, got 95"):
        H.logits(x[:95])
    out, buf = C.c_void_p(), np.zeros(10, np.float32)
    with pytest.raises(KernelError, match=r"lm_head is 10 floats; expected 3x4 = 12"):
        _lib.check(_lib.load().qbk_head_create(ctx.handle, buf.ctypes.data, 10, 3, 4, C.byref(out)))
    H.close()
