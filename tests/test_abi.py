"""C-ABI checks that need no GPU: libqbk.so loads, exports every symbol
include/qbk.h declares, its host-side functions agree with the oracle and the
reference's error texts, and device init fails closed with the hint when no
device is visible (gpu.rs:85-101)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from conftest import ROOT


@pytest.fixture(scope="module")
def lib():
    from quantibbler_amd import _lib

    return _lib.load()


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "qbk.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qbk_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), f"libqbk.so does not export {n}"
    from quantibbler_amd import _lib

    assert set(_lib.EXPORTED) <= set(names) | {"qbk_backend_version", "qbk_last_error"}


def test_library_is_gfx950_code_object():
    so = os.path.join(ROOT, "quantibbler_amd", "libqbk.so")
    blob = open(so, "rb").read()
    assert b"gfx950" in blob


def test_host_bit_layout_matches_oracle(orc):
    from quantibbler_amd import kernels as K

    rng = np.random.default_rng(2)
    for rows, cols in [(5, 11), (3, 64), (7, 1), (1, 129)]:
        f = rng.choice([-1, 1], (rows, cols)).astype(np.int8)
        p = K.pack_bits(f)
        assert p.tobytes() == orc.pack_bits(f).tobytes()
        assert K.unpack_bits(p, cols, "int8").tobytes() == f.tobytes()
        assert K.unpack_bits(p, cols, "float64").tolist() == f.astype(np.float64).tolist()
    x = np.array([0.0, -0.0, 1.5, -2.5, -1e-9, 1e-300])
    assert K.sign_estimate(x).tolist() == orc.sign_estimate(x).tolist()


def test_host_error_texts():
    from quantibbler_amd import KernelError
    from quantibbler_amd import kernels as K

    with pytest.raises(KernelError, match=r"pack_bits expects values in \{-1, \+1\}; got 0.5"):
        K.pack_bits(np.array([[1.0, 0.5]]))
    with pytest.raises(KernelError, match=r"n_bits=17 exceeds the packed width 2 \(16 bits\)"):
        K.unpack_bits(np.zeros((1, 2), np.uint8), 17, "int8")
    with pytest.raises(KernelError, match="packed length 2 does not match 1 rows x 1 bitplanes"):
        K.unpack_bits(np.zeros((1, 2), np.uint8), 8, "int8")
    with pytest.raises(KernelError, match="unpack_bits dtype must be 'int8' or 'float64', got \"float32\""):
        K.unpack_bits(np.zeros((1, 1), np.uint8), 8, "float32")
    with pytest.raises(KernelError, match=r'unknown kernel dtype "float16"; expected one of "float64", "float32", "bfloat16"'):
        K.packed_matvec_dtype(np.zeros((1, 1), np.uint8), 8, np.zeros(8), "float16")


def test_validation_precedes_device_use(lib):
    # shape errors are reported before any device is touched (gpu.rs:123-137)
    from quantibbler_amd import KernelError
    from quantibbler_amd._lib import check

    packed, vec, out = np.zeros(2, np.uint8), np.zeros(8), np.zeros(1)
    with pytest.raises(KernelError, match="vec must have length 9, got 8"):
        check(lib.qbk_packed_matvec(None, 0, packed.ctypes.data, 2, 1, 9, vec.ctypes.data, 8,
                                    out.ctypes.data))
    with pytest.raises(KernelError, match="packed length 2 does not match 3 rows x 2 bitplanes"):
        check(lib.qbk_packed_matvec(None, 0, packed.ctypes.data, 2, 3, 9, vec.ctypes.data, 9,
                                    out.ctypes.data))
    with pytest.raises(KernelError, match="sage attention requires a positive block_size"):
        from quantibbler_amd._lib import AttnShape

        sh = AttnShape(1, 2, 1, 8, 8, 4, 4)
        check(lib.qbk_attention_sage(None, C.byref(sh), None, 64, None, 32, None, 32, 1, 0, None))
    with pytest.raises(KernelError, match=r"n_kv_heads must divide n_heads: n_heads=3, n_kv_heads=2"):
        sh = AttnShape(1, 3, 2, 8, 8, 4, 4)
        check(lib.qbk_attention_sage(None, C.byref(sh), None, 0, None, 0, None, 0, 1, 4, None))
    with pytest.raises(KernelError, match=r"query must hold 64 values for AttentionShape \{ batch: 1, "
                       r"n_heads: 2, n_kv_heads: 1, seq_q: 8, seq_kv: 8, head_dim: 4, val_dim: 4 \}, got 63"):
        sh = AttnShape(1, 2, 1, 8, 8, 4, 4)
        check(lib.qbk_attention_sage(None, C.byref(sh), None, 63, None, 32, None, 32, 1, 4, None))


def test_block_attention_face_validation(lib):
    # the face setter validates before it touches a block (engine/mod.rs:953-968
    # knows three faces; the device block serves the sage and exact ones)
    from quantibbler_amd import KernelError
    from quantibbler_amd._lib import check

    with pytest.raises(KernelError, match="null block"):
        check(lib.qbk_block_set_attention_face(None, 1))
    with pytest.raises(KernelError, match="null block"):
        check(lib.qbk_block_set_serving(None, None, 1))


def test_packed_matvec_ceiling_precedes_device_use(lib):
    # gpu.rs:116-137: after validate_packed and the vec length check, the f64
    # device face refuses n_rows x words past the u32 index ceiling -- before
    # any device use, so no context is needed and nothing is read
    from quantibbler_amd import KernelError
    from quantibbler_amd._lib import check

    vec = (C.c_double * 8)()
    rows = 1 << 32                      # 2^32 rows x 1 word: lengths match, past the ceiling
    with pytest.raises(KernelError, match=r"^packed shape 4294967296 x 1 words exceeds the device u32 index "
                                          r"ceiling \(4294967295\); use the CPU rlib face$"):
        check(lib.qbk_packed_matvec(None, 0, None, rows, rows, 8, vec, 8, None))
    rows = (1 << 30) + 1                # 2^30 + 1 rows x 4 words: the product passes it
    with pytest.raises(KernelError, match=r"^packed shape 1073741825 x 4 words exceeds the device u32"):
        check(lib.qbk_packed_matvec(None, 0, None, 4 * rows, rows, 32, (C.c_double * 32)(), 32, None))
    # the shape checks come first, with their own texts
    with pytest.raises(KernelError, match=r"^packed length 5 does not match 4294967296 rows x 1 bitplanes$"):
        check(lib.qbk_packed_matvec(None, 0, None, 5, 1 << 32, 8, vec, 8, None))
    with pytest.raises(KernelError, match=r"^vec must have length 8, got 7$"):
        check(lib.qbk_packed_matvec(None, 0, None, 1 << 32, 1 << 32, 8, vec, 7, None))
    # the ceiling is the f64 device face's: f32 / bf16 (core.rs's faces) have none,
    # so at this shape they go on to the device (not called here)


def test_exact_attention_validation_and_ceiling_precede_device_use(lib):
    # gpu_attention.rs:466-509: the exact face's messages, then its u32
    # index ceiling -- both before any device is touched
    from quantibbler_amd import KernelError
    from quantibbler_amd._lib import AttnShape, check

    with pytest.raises(KernelError, match="n_kv_heads must divide n_heads: n_heads=3, n_kv_heads=2"):
        sh = AttnShape(1, 3, 2, 8, 8, 4, 4)
        check(lib.qbk_attention(None, C.byref(sh), None, 0, None, 0, None, 0, 1, None))
    with pytest.raises(KernelError, match=r"key must hold 32 values for AttentionShape \{ batch: 1, "
                       r"n_heads: 2, n_kv_heads: 1, seq_q: 8, seq_kv: 8, head_dim: 4, val_dim: 4 \}, got 31"):
        sh = AttnShape(1, 2, 1, 8, 8, 4, 4)
        check(lib.qbk_attention(None, C.byref(sh), None, 64, None, 31, None, 32, 1, None))
    big = 1 << 31   # 2^31 keys x 4 channels: past the u32 ceiling; lengths match, nothing is read
    sh = AttnShape(1, 1, 1, 1, big, 4, 4)
    with pytest.raises(KernelError, match=r"attention inputs exceed the device u32 index ceiling \(4294967295\); "
                                          "use the CPU reference face"):
        check(lib.qbk_attention(None, C.byref(sh), None, 4, None, 4 * big, None, 4 * big, 0, None))
    with pytest.raises(KernelError, match=r"sage attention inputs exceed the device u32 index ceiling"):
        sh = AttnShape(1, 1, 1, big, big, 4, 4)
        check(lib.qbk_attention_sage(None, C.byref(sh), None, 4 * big, None, 4 * big, None, 4 * big, 0, 64,
                                     None))


def test_decode_validation_precedes_device_use(lib):
    # the decode step's shape checks (batch 1, one query, the cache's sizes)
    # are reported before any device is touched
    from quantibbler_amd import KernelError
    from quantibbler_amd._lib import AttnShape, check

    def call(sh, lens, block=4):
        return check(lib.qbk_attention_sage_decode(None, C.byref(sh), None, lens[0], None, lens[1],
                                                   None, lens[2], block, None, lens[3]))

    with pytest.raises(KernelError, match="sage decode takes one sequence: batch must be 1, got 2"):
        call(AttnShape(2, 2, 1, 1, 8, 4, 4), (8, 32, 32, 8))
    with pytest.raises(KernelError, match="sage decode takes the step's one query: seq_q must be 1, got 8"):
        call(AttnShape(1, 2, 1, 8, 8, 4, 4), (8, 32, 32, 8))
    with pytest.raises(KernelError, match=r"n_kv_heads must divide n_heads: n_heads=3, n_kv_heads=2"):
        call(AttnShape(1, 3, 2, 1, 8, 4, 4), (12, 64, 64, 12))
    with pytest.raises(KernelError, match="sage attention requires a positive block_size"):
        call(AttnShape(1, 2, 1, 1, 8, 4, 4), (8, 32, 32, 8), block=0)
    with pytest.raises(KernelError, match=r"key cache must hold 32 values for AttentionShape \{ batch: 1, "
                       r"n_heads: 2, n_kv_heads: 1, seq_q: 1, seq_kv: 8, head_dim: 4, val_dim: 4 \}, got 31"):
        call(AttnShape(1, 2, 1, 1, 8, 4, 4), (8, 31, 32, 8))
    with pytest.raises(KernelError, match="out must hold 8 values"):
        call(AttnShape(1, 2, 1, 1, 8, 4, 4), (8, 32, 32, 7))
    assert lib.qbk_sage_decode_workspace_size(C.byref(AttnShape(1, 2, 1, 1, 8, 4, 4)), 4) > 0


def test_decode_state_validation_precedes_device_use(lib):
    # the kept-state step checks its capacity, cached count and state size
    # before any device is touched
    from quantibbler_amd import KernelError
    from quantibbler_amd._lib import AttnShape, check

    sh = AttnShape(1, 2, 1, 1, 8, 4, 4)
    need = lib.qbk_sage_decode_workspace_size(C.byref(AttnShape(1, 2, 1, 1, 4096, 4, 4)), 4)
    assert need > lib.qbk_sage_decode_workspace_size(C.byref(sh), 4)

    def call(cap, cached, size=need, shape=sh):
        return check(lib.qbk_attention_sage_decode_step_dev(None, C.byref(shape), None, None, None, 4, None,
                                                            None, size, cap, cached, None))

    with pytest.raises(KernelError, match="the cache holds 8 tokens, beyond the state's capacity of 7"):
        call(7, 0)
    with pytest.raises(KernelError, match=r"cached_tokens \(9\) exceeds the 8 tokens of the cache"):
        call(4096, 9)
    with pytest.raises(KernelError, match=f"decode state of {need - 1} bytes is smaller than the {need} "
                       "a capacity of 4096 tokens needs"):
        call(4096, 8, need - 1)
    with pytest.raises(KernelError, match="sage decode takes the step's one query"):
        call(4096, 0, shape=AttnShape(1, 2, 1, 2, 8, 4, 4))
    with pytest.raises(KernelError, match="null buffer"):
        call(4096, 8)


def test_init_fails_closed_without_device(lib):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        pytest.skip("a device is visible; the fail-closed path is exercised on CPU hosts")
    from quantibbler_amd import GpuContext, InitError, gpu_available

    assert gpu_available() is False
    with pytest.raises(InitError, match="no usable HIP/ROCm device"):
        GpuContext(0)


def header_arities():
    """Each function include/qbk.h declares and its parameter count."""
    text = open(os.path.join(ROOT, "include", "qbk.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(qbk_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_rust_binding_declares_only_exported_symbols(lib):
    """quantibbler_amd/rust/qbk-sys declares the C ABI for the reference's
    Rust side (no cargo here to build it): it binds every function
    include/qbk.h declares, each with the header's parameter count, all
    exported by libqbk.so, and its struct mirror of AttentionShape has the
    header's field order."""
    src = open(os.path.join(ROOT, "quantibbler_amd", "rust", "qbk-sys", "src", "lib.rs")).read()
    bound = dict(re.findall(r"pub fn (qbk_[a-z0-9_]+)\(([^)]*)\)", src))
    declared = header_arities()
    assert set(bound) == set(declared), sorted(set(bound) ^ set(declared))
    for n, args in sorted(bound.items()):
        assert hasattr(lib, n), f"{n} is not exported"
        assert (args.count(":") if args.strip() else 0) == declared[n], f"{n}: parameter count differs from qbk.h"
    fields = re.search(r"pub struct AttentionShape \{(.*?)\}", src, re.S).group(1)
    assert re.findall(r"pub (\w+): usize", fields) == ["batch", "n_heads", "n_kv_heads", "seq_q", "seq_kv",
                                                       "head_dim", "val_dim"]


def test_driver_scripts_compile():
    """bench.py and __graft_entry__.py, which the driver runs on the GPU box,
    at least compile here."""
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for name in ("bench.py", "__graft_entry__.py"):
        with open(os.path.join(root, name)) as f:
            compile(f.read(), name, "exec")
