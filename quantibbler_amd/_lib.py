"""ctypes loader for libqbk.so (the HIP library) and its C-ABI signatures.

The library is required: importing the package without a built libqbk.so
raises, and every device call fails loudly when no MI355X is usable.  There
is no CPU fallback for any device entry point.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqbk.so")

QBK_OK, QBK_ERR_VALIDATION, QBK_ERR_DEVICE, QBK_ERR_INIT = 0, 1, 2, 3
QBK_F64, QBK_F32, QBK_BF16 = 0, 1, 2


class KernelError(ValueError):
    """core::KernelError (core.rs:31): a validation failure, reference text."""


class DeviceError(RuntimeError):
    """A HIP call failed during a device call (gpu.rs: per-call hard error)."""


class InitError(RuntimeError):
    """No usable device (gpu.rs GpuContext::init_at failure)."""


class AttnShape(C.Structure):
    """gpu_attention.rs:402-411 AttentionShape."""
    _fields_ = [(n, C.c_size_t) for n in
                ("batch", "n_heads", "n_kv_heads", "seq_q", "seq_kv", "head_dim", "val_dim")]


_P, _Z, _I = C.c_void_p, C.c_size_t, C.c_int
_SIGS = {
    "qbk_backend_version": (C.c_char_p, []),
    "qbk_last_error": (C.c_char_p, []),
    "qbk_dtype_from_name": (_I, [C.c_char_p, C.POINTER(C.c_int)]),
    "qbk_pack_bits": (_I, [_P, _Z, _Z, _Z, _P]),
    "qbk_unpack_bits": (_I, [_P, _Z, _Z, _Z, _P]),
    "qbk_validate_packed": (_I, [_Z, _Z, _Z, C.POINTER(C.c_size_t)]),
    "qbk_sign_estimate": (None, [_P, _Z, _P]),
    "qbk_joint_itq": (_I, [_P, _Z, _P, _Z, _Z, _Z, _Z, _Z, C.c_double, C.c_uint64, _P, _P, C.POINTER(_Z),
                           C.POINTER(_I)]),
    "qbk_ctx_create": (_I, [_I, C.POINTER(_P)]),
    "qbk_ctx_destroy": (None, [_P]),
    "qbk_gpu_available": (_I, []),
    "qbk_packed_matvec": (_I, [_P, _I, _P, _Z, _Z, _Z, _P, _Z, _P]),
    "qbk_packed_matmul": (_I, [_P, _I, _P, _Z, _Z, _Z, _P, _Z, _Z, _P]),
    "qbk_packed_matvec_dev": (_I, [_P, _I, _P, _Z, _Z, _P, _P, _P]),
    "qbk_packed_matmul_dev": (_I, [_P, _I, _P, _Z, _Z, _P, _Z, _Z, _P, _P]),
    "qbk_factor_from_qpk1": (_I, [_P, _P, _Z, C.POINTER(_P)]),
    "qbk_factor_from_rows": (_I, [_P, _Z, _Z, _Z, _P, _P, _P, _P, _P, C.POINTER(_P)]),
    "qbk_factor_destroy": (None, [_P]),
    "qbk_factor_dims": (_I, [_P, C.POINTER(_Z), C.POINTER(_Z), C.POINTER(_Z)]),
    "qbk_factor_workspace_size": (_Z, [_P, _Z]),
    "qbk_factor_linear_dev": (_I, [_P, _P, _P, _Z, _P, _I, _P, _Z, _P]),
    "qbk_factor_apply": (_I, [_P, _P, _I, _P, _Z, _P]),
    "qbk_factor_linear_noalloc_dev": (_I, [_P, _P, _P, _Z, _P, _I, _P]),
    "qbk_factor_set_create": (_I, [_P, _P, _Z, C.POINTER(_P)]),
    "qbk_factor_set_destroy": (None, [_P]),
    "qbk_factor_set_workspace_size": (_Z, [_P]),
    "qbk_factor_set_decode_dev": (_I, [_P, _P, _P, _P, _P, _Z, _P]),
    "qbk_factor_set_workspace_size_batch": (_Z, [_P, _Z]),
    "qbk_factor_set_decode_batch_dev": (_I, [_P, _P, _Z, _P, _P, _P, _Z, _P]),
    "qbk_factor_set_shared_workspace_size": (_Z, [_P, _Z]),
    "qbk_factor_set_shared_dev": (_I, [_P, _P, _Z, _P, _P, _P, _Z, _P]),
    "qbk_factor_set_stage_dev": (_I, [_P, _P, _I, _P, _P, _P, _Z, _P]),
    "qbk_attention": (_I, [_P, C.POINTER(AttnShape), _P, _Z, _P, _Z, _P, _Z, _I, _P]),
    "qbk_attention_dev": (_I, [_P, C.POINTER(AttnShape), _P, _P, _P, _I, _P, _P]),
    "qbk_attention_sage": (_I, [_P, C.POINTER(AttnShape), _P, _Z, _P, _Z, _P, _Z, _I, _Z, _P]),
    "qbk_attention_sage_dev": (_I, [_P, C.POINTER(AttnShape), _P, _P, _P, _I, _Z, _P, _P]),
    "qbk_attention_sage_decode": (_I, [_P, C.POINTER(AttnShape), _P, _Z, _P, _Z, _P, _Z, _Z, _P, _Z]),
    "qbk_sage_decode_workspace_size": (_Z, [C.POINTER(AttnShape), _Z]),
    "qbk_attention_sage_decode_dev": (_I, [_P, C.POINTER(AttnShape), _P, _P, _P, _Z, _P, _P, _Z, _P]),
    "qbk_block_create": (_I, [_P, _P, _P, _Z, _P, _Z, _P, _P, _Z, _Z, _Z, _Z, C.c_double, C.c_double, _Z, _Z,
                              _P]),
    "qbk_embed": (_I, [_P, _P, _Z, _Z, _P, _Z, _P, _P]),
    "qbk_embed_dev": (_I, [_P, _P, _Z, _Z, _P, _Z, _P, _P]),
    "qbk_rms_norm_dev": (_I, [_P, _P, _Z, _Z, _P, C.c_double, _P, _P]),
    "qbk_rms_norm_f32_dev": (_I, [_P, _P, _Z, _Z, _P, C.c_double, _P, _P]),
    "qbk_argmax_dev": (_I, [_P, _P, _Z, _Z, _P, _P]),
    "qbk_block_destroy": (None, [_P]),
    "qbk_block_decode_dev": (_I, [_P, _P, _P, _Z, _P]),
    "qbk_block_reset": (_I, [_P]),
    "qbk_block_prefill_workspace_size": (_Z, [_P, _Z]),
    "qbk_block_prefill_dev": (_I, [_P, _P, _P, _Z, _P, _Z, _P]),
    "qbk_block_cache": (_I, [_P, _P, _P]),
    "qbk_block_create_seqs": (_I, [_P, _P, _P, _Z, _P, _Z, _P, _P, _Z, _Z, _Z, _Z, C.c_double, C.c_double, _Z,
                                   _Z, _Z, _P]),
    "qbk_block_prefill_seq_dev": (_I, [_P, _P, _Z, _P, _Z, _P, _Z, _P]),
    "qbk_block_decode_batch_workspace_size": (_Z, [_P, _Z]),
    "qbk_block_decode_batch_dev": (_I, [_P, _P, _P, _P, _Z, _P, _Z, _P]),
    "qbk_block_decode_pos_dev": (_I, [_P, _P, _P, _P, _P]),
    "qbk_block_decode_batch_pos_dev": (_I, [_P, _P, _P, _P, _Z, _P, _Z, _P]),
    "qbk_block_set_positions": (_I, [_P, _P, _Z]),
    "qbk_block_set_filled": (_I, [_P, _P, _Z]),
    "qbk_block_set_attention_face": (_I, [_P, _I]),
    "qbk_block_set_serving": (_I, [_P, _P, _I]),
    "qbk_positions_advance_dev": (_I, [_P, _P, _Z, _P]),
    "qbk_attention_sage_decode_step_dev": (_I, [_P, C.POINTER(AttnShape), _P, _P, _P, _Z, _P, _P, _Z, _Z,
                                                _Z, _P]),
    "qbk_head_create": (_I, [_P, _P, _Z, _Z, _Z, C.POINTER(_P)]),
    "qbk_head_create_dev": (_I, [_P, _P, _Z, _Z, C.POINTER(_P)]),
    "qbk_head_destroy": (None, [_P]),
    "qbk_head_info": (_I, [_P, C.POINTER(_Z), C.POINTER(_Z), C.POINTER(_I)]),
    "qbk_head_logits": (_I, [_P, _P, _P, _Z, _P, _Z]),
    "qbk_head_logits_dev": (_I, [_P, _P, _P, _Z, _P, _P]),
    "qbk_sage_blk_workspace_size": (_Z, [C.POINTER(AttnShape)]),
    "qbk_attention_sage_blk_dev": (_I, [_P, C.POINTER(AttnShape), _P, _P, _P, _I, _P, _P, _Z, _P]),
    "qbk_sage_blk_quantize_dev": (_I, [_P, C.POINTER(AttnShape), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
}

EXPORTED = tuple(_SIGS)

_lib = None


def load():
    """Load libqbk.so once; raises ImportError if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libqbk.so not found at {LIB_PATH}; build it with "
                "`python quantibbler_amd/build.py` (hipcc, gfx950)")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    """Map a QBK_* status to the matching Python exception."""
    if rc == QBK_OK:
        return
    msg = load().qbk_last_error().decode()
    if rc == QBK_ERR_VALIDATION:
        raise KernelError(msg)
    if rc == QBK_ERR_INIT:
        raise InitError(msg)
    raise DeviceError(msg)
