"""ctypes face of the C oracle (oracle/qbk_oracle.c) — TEST INFRASTRUCTURE ONLY.

NumPy in, NumPy out.  Each wrapper names the reference function whose
arithmetic the C code restates; see qbk_oracle.c for the citations and for
what pins each function.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liborc.so")
_lib = None


class OracleError(ValueError):
    """A validation error raised by the oracle, carrying the reference's text."""


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc); returns the .so path."""
    if force or not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = C.CDLL(_SO)
        _declare(_lib)
    return _lib


class AttnShape(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in
                ("batch", "n_heads", "n_kv_heads", "seq", "head_dim", "val_dim")]


class Qpk1Header(C.Structure):
    _fields_ = [("version", C.c_uint32), ("dtype_tag", C.c_uint32)] + [
        (n, C.c_size_t) for n in
        ("dout", "din", "r", "s1_off", "s2_off", "bias_off", "ub_off", "vb_off")]


_P = C.c_void_p
_Z = C.c_size_t


def _declare(L):
    sig = {
        "orc_pack_bits": (C.c_int, [_P, _Z, _Z, _Z, _P, C.c_char_p, _Z]),
        "orc_unpack_bits": (C.c_int, [_P, _Z, _Z, _Z, _P, C.c_char_p, _Z]),
        "orc_validate_packed": (C.c_int, [_Z, _Z, _Z, _P, C.c_char_p, _Z]),
        "orc_sign_estimate": (None, [_P, _Z, _P]),
        "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_packed_matvec": (C.c_int, [C.c_int, _P, _Z, _Z, _Z, _P, _Z, _P, C.c_char_p, _Z]),
        "orc_packed_matmul": (C.c_int, [C.c_int, _P, _Z, _Z, _Z, _P, _Z, _Z, _P, C.c_char_p, _Z]),
        "orc_fast_packed_matvec_f64": (C.c_int, [_P, _Z, _Z, _Z, _P, _Z, _P, C.c_int, C.c_char_p, _Z]),
        "orc_fast_packed_matmul_f64": (C.c_int, [_P, _Z, _Z, _Z, _P, _Z, _Z, _P, C.c_int, C.c_char_p, _Z]),
        "orc_qpk1_parse": (C.c_int, [_P, _Z, C.POINTER(Qpk1Header), _P, _P, _P, C.c_char_p, _Z]),
        "orc_qpk1_expected_size": (_Z, [_Z, _Z, _Z, C.c_int, C.c_int]),
        "orc_container_to_rows": (None, [_P, _Z, _Z, _P]),
        "orc_container_to_rows_transposed": (None, [_P, _Z, _Z, _P]),
        "orc_factor_apply": (C.c_int, [C.c_int, _Z, _Z, _Z, _P, _P, _P, _P, _P, _P, _P, C.c_int, C.c_int]),
        "orc_factor_apply_bf16_batch": (None, [_Z, _Z, _Z, _P, _P, _P, _P, _P, _P, _Z, _P, _P, C.c_int]),
        "orc_attention_tiled_f64": (C.c_int, [C.POINTER(AttnShape), _P, _P, _P, C.c_int, _Z, _P, _P]),
        "orc_attention_sage_np_f64": (C.c_int, [C.POINTER(AttnShape), _P, _P, _P, C.c_int, _Z, _P]),
        "orc_attention_sage_dev_f32": (C.c_int, [C.POINTER(AttnShape), _P, _P, _P, C.c_int, _Z, _P, _P, _P, C.c_int]),
        "orc_expf": (C.c_float, [C.c_float]),
        "orc_attention_sage_blk": (C.c_int, [C.POINTER(AttnShape), _P, _P, _P, C.c_int, _P, _P, _P, _P, _P, _P, C.c_int]),
        "orc_head_logits": (None, [_P, _Z, _Z, _P, _Z, _P, C.c_int]),
        "orc_rms_norm_f32": (None, [_P, _P, _Z, C.c_double, _P]),
        "orc_rope_rotate": (None, [_P, _Z, _Z, _Z, C.c_double]),
        "orc_gqa_attention_scalar": (None, [_P, _P, _P, _Z, _Z, _Z, _Z, _P, _P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _ptr(a):
    return None if a is None else a.ctypes.data


def _err():
    return C.create_string_buffer(512)


def _check(rc, err):
    if rc != 0:
        raise OracleError(err.value.decode())


def _threads(threads):
    return threads if threads else (os.cpu_count() or 1)


# ---- bit layout (core.rs:129-240) ------------------------------------------

def pack_bits(factor) -> np.ndarray:
    f = np.ascontiguousarray(factor, dtype=np.int8)
    rows = int(np.prod(f.shape[:-1], dtype=np.int64)) if f.ndim > 1 else 1
    cols = f.shape[-1]
    out = np.zeros((rows, (cols + 7) // 8), dtype=np.uint8)
    e = _err()
    _check(lib().orc_pack_bits(_ptr(f), f.size, rows, cols, _ptr(out), e, 512), e)
    return out


def unpack_bits(packed, n_bits: int, n_rows=None) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    rows = n_rows if n_rows is not None else (p.shape[0] if p.ndim == 2 else 1)
    out = np.zeros((rows, n_bits), dtype=np.int8)
    e = _err()
    _check(lib().orc_unpack_bits(_ptr(p), p.size, rows, n_bits, _ptr(out), e, 512), e)
    return out


def validate_packed(packed_len: int, n_rows: int, n_bits: int) -> int:
    w = C.c_size_t(0)
    e = _err()
    _check(lib().orc_validate_packed(packed_len, n_rows, n_bits, C.byref(w), e, 512), e)
    return w.value


def sign_estimate(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float64).ravel()
    out = np.zeros(a.size, dtype=np.int8)
    lib().orc_sign_estimate(_ptr(a), a.size, _ptr(out))
    return out


def f32_to_bf16(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().orc_f32_to_bf16
    return np.array([f(float(v)) for v in a.ravel()], dtype=np.uint16).reshape(a.shape)


def f32_to_bf16_fast(x) -> np.ndarray:
    """Vectorised RNE (same rule as orc_f32_to_bf16 for non-NaN input)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    return (((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) & np.uint64(0xFFFF)).astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# ---- products (core.rs:202-317; fast.rs:28-158) ------------------------------

_DT = {"float64": (0, np.float64), "float32": (1, np.float32), "bfloat16": (2, np.uint16)}


def packed_matvec(packed, n_rows: int, n_bits: int, vec, dtype: str = "float64"):
    code, npdt = _DT[dtype]
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    v = np.ascontiguousarray(vec, dtype=npdt).ravel()
    out = np.zeros(n_rows, dtype=npdt)
    e = _err()
    _check(lib().orc_packed_matvec(code, _ptr(p), p.size, n_rows, n_bits, _ptr(v), v.size,
                                   _ptr(out), e, 512), e)
    return out


def packed_matmul(packed, n_rows: int, n_bits: int, mat, n_cols: int, dtype: str = "float64"):
    code, npdt = _DT[dtype]
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    m = np.ascontiguousarray(mat, dtype=npdt).ravel()
    kc = m.size // max(n_bits, 1)
    out = np.zeros(n_rows * kc, dtype=npdt)
    e = _err()
    _check(lib().orc_packed_matmul(code, _ptr(p), p.size, n_rows, n_bits, _ptr(m), m.size,
                                   n_cols, _ptr(out), e, 512), e)
    return out.reshape(n_rows, kc)


def fast_packed_matvec(packed, n_rows: int, n_bits: int, vec, threads: int = 0):
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    v = np.ascontiguousarray(vec, dtype=np.float64).ravel()
    out = np.zeros(n_rows, dtype=np.float64)
    e = _err()
    _check(lib().orc_fast_packed_matvec_f64(_ptr(p), p.size, n_rows, n_bits, _ptr(v), v.size,
                                            _ptr(out), _threads(threads), e, 512), e)
    return out


def fast_packed_matmul(packed, n_rows: int, n_bits: int, mat, n_cols: int, threads: int = 0):
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    m = np.ascontiguousarray(mat, dtype=np.float64).ravel()
    kc = m.size // max(n_bits, 1)
    out = np.zeros(n_rows * kc, dtype=np.float64)
    e = _err()
    _check(lib().orc_fast_packed_matmul_f64(_ptr(p), p.size, n_rows, n_bits, _ptr(m), m.size,
                                            n_cols, _ptr(out), _threads(threads), e, 512), e)
    return out.reshape(n_rows, kc)


# ---- qpk1 + engine layout (qpk1 lib.rs:152-320; engine/mod.rs:258-481) ------

def qpk1_parse(stream: bytes) -> dict:
    b = np.frombuffer(stream, dtype=np.uint8).copy()
    hdr = Qpk1Header()
    e = _err()
    _check(lib().orc_qpk1_parse(_ptr(b), b.size, C.byref(hdr), None, None, None, e, 512), e)
    s1 = np.zeros(hdr.dout, np.float64)
    s2 = np.zeros(hdr.din, np.float64)
    bias = np.zeros(hdr.dout, np.float64)
    _check(lib().orc_qpk1_parse(_ptr(b), b.size, C.byref(hdr), _ptr(s1), _ptr(s2), _ptr(bias),
                                e, 512), e)
    ub_len = (hdr.dout * hdr.r + 7) // 8
    vb_len = (hdr.din * hdr.r + 7) // 8
    return {
        "version": hdr.version, "dtype_tag": hdr.dtype_tag, "dout": hdr.dout, "din": hdr.din,
        "r": hdr.r, "s1": s1, "s2": s2, "bias": bias if hdr.version >= 2 else np.zeros(0),
        "ub_packed": b[hdr.ub_off:hdr.ub_off + ub_len].copy(),
        "vb_packed": b[hdr.vb_off:hdr.vb_off + vb_len].copy(),
    }


def qpk1_layer(stream: bytes) -> dict:
    """crates/quantibbler-qpk1/src/lib.rs:229-320 parse, then
    engine/mod.rs:342-381 PackedLayer::from_layer: the per-row bitplanes
    (container_to_rows / _transposed) and the f32 scales (f16 and f32 widen
    exactly; a v1 layer's bias is the zero map)."""
    L = qpk1_parse(stream)
    dout, din, r = L["dout"], L["din"], L["r"]
    bias = L["bias"] if L["bias"].size else np.zeros(dout)
    return dict(dout=dout, din=din, r=r, version=L["version"], dtype_tag=L["dtype_tag"],
                ub=container_to_rows(L["ub_packed"], dout, r),
                vt=container_to_rows_transposed(L["vb_packed"], din, r),
                s1=L["s1"].astype(np.float32), s2=L["s2"].astype(np.float32),
                bias=bias.astype(np.float32))


def qpk1_expected_size(dout, din, r, itemsize, with_bias) -> int:
    return lib().orc_qpk1_expected_size(dout, din, r, itemsize, int(with_bias))


def container_to_rows(packed, n_rows: int, r: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(n_rows * ((r + 7) // 8), np.uint8)
    lib().orc_container_to_rows(_ptr(p), n_rows, r, _ptr(out))
    return out


def container_to_rows_transposed(packed, din: int, r: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(r * ((din + 7) // 8), np.uint8)
    lib().orc_container_to_rows_transposed(_ptr(p), din, r, _ptr(out))
    return out


def factor_apply(serving: str, dout, din, r, ub_rows, vb_t_rows, s1, s2, bias, x,
                 fast: bool = False, threads: int = 0) -> np.ndarray:
    """engine/mod.rs:393-481 PackedLayer::apply ("fp32") / apply_bf16 ("bf16")."""
    ub = np.ascontiguousarray(ub_rows, np.uint8)
    vt = np.ascontiguousarray(vb_t_rows, np.uint8)
    a1 = np.ascontiguousarray(s1, np.float32)
    a2 = np.ascontiguousarray(s2, np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    xx = np.ascontiguousarray(x, np.float32)
    y = np.zeros(dout, np.float32)
    rc = lib().orc_factor_apply(0 if serving == "fp32" else 1, dout, din, r, _ptr(ub), _ptr(vt),
                                _ptr(a1), _ptr(a2), _ptr(bb), _ptr(xx), _ptr(y), int(fast),
                                _threads(threads))
    if rc:
        raise OracleError("factor_apply failed")
    return y


def factor_apply_bf16_batch(dout, din, r, ub_rows, vb_t_rows, s1, s2, bias, x_bf16,
                            threads: int = 0, want_t: bool = False):
    """Token-major batched apply_bf16; returns y f32 [batch, dout] (and t bf16)."""
    ub = np.ascontiguousarray(ub_rows, np.uint8)
    vt = np.ascontiguousarray(vb_t_rows, np.uint8)
    a1 = np.ascontiguousarray(s1, np.float32)
    a2 = np.ascontiguousarray(s2, np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    x = np.ascontiguousarray(x_bf16, np.uint16)
    batch = x.size // din
    y = np.zeros((batch, dout), np.float32)
    t = np.zeros((batch, r), np.uint16) if want_t else None
    lib().orc_factor_apply_bf16_batch(dout, din, r, _ptr(ub), _ptr(vt), _ptr(a1), _ptr(a2),
                                      _ptr(bb), _ptr(x), batch, _ptr(y), _ptr(t),
                                      _threads(threads))
    return (y, t) if want_t else y


# ---- attention --------------------------------------------------------------

def _shape(q, k, v):
    b, h, s, d = q.shape
    return AttnShape(b, h, k.shape[1], s, d, v.shape[3])


def attention_tiled(q, k, v, causal=False, block_size=64, return_lse=False):
    """attention_tiled.py:76-180 (exact, f64)."""
    q = np.ascontiguousarray(q, np.float64)
    k = np.ascontiguousarray(k, np.float64)
    v = np.ascontiguousarray(v, np.float64)
    sh = _shape(q, k, v)
    out = np.zeros(q.shape[:3] + (v.shape[3],), np.float64)
    lse = np.zeros(q.shape[:3], np.float64)
    lib().orc_attention_tiled_f64(C.byref(sh), _ptr(q), _ptr(k), _ptr(v), int(causal),
                                  block_size, _ptr(out), _ptr(lse))
    return (out, lse) if return_lse else out


def attention_sage_np(q, k, v, causal=False, block_size=64):
    """attention_sage.py:206-350 (f64 NumPy semantics)."""
    q = np.ascontiguousarray(q, np.float64)
    k = np.ascontiguousarray(k, np.float64)
    v = np.ascontiguousarray(v, np.float64)
    sh = _shape(q, k, v)
    out = np.zeros(q.shape[:3] + (v.shape[3],), np.float64)
    lib().orc_attention_sage_np_f64(C.byref(sh), _ptr(q), _ptr(k), _ptr(v), int(causal),
                                    block_size, _ptr(out))
    return out


def attention_sage_dev(q, k, v, causal=False, block_size=64, threads=0, stages=False):
    """gpu_attention.rs:89-396 (f32 device semantics, orc_expf)."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    sh = _shape(q, k, v)
    out = np.zeros(q.shape[:3] + (v.shape[3],), np.float32)
    qhat = np.zeros(q.shape, np.int8) if stages else None
    qd = np.zeros(q.shape[:3], np.float32) if stages else None
    lib().orc_attention_sage_dev_f32(C.byref(sh), _ptr(q), _ptr(k), _ptr(v), int(causal),
                                     block_size, _ptr(out), _ptr(qhat), _ptr(qd),
                                     _threads(threads))
    return (out, qhat, qd) if stages else out


def expf(x: float) -> float:
    return lib().orc_expf(float(x))


def attention_sage_blk(q_bf16, k_bf16, v_bf16, causal=True, threads=0, stages=False):
    """Block-scaled Sage variant (north_star scheme).  Inputs are bf16 bit
    patterns (uint16) shaped (B,H,S,d)/(B,Hkv,S,d)/(B,Hkv,S,dv)."""
    q = np.ascontiguousarray(q_bf16, np.uint16)
    k = np.ascontiguousarray(k_bf16, np.uint16)
    v = np.ascontiguousarray(v_bf16, np.uint16)
    sh = _shape(q, k, v)
    B, H, S, d = q.shape
    Hk = k.shape[1]
    nblk = (S + 63) // 64
    out = np.zeros(q.shape[:3] + (v.shape[3],), np.float32)
    st = None
    if stages:
        st = {
            "qhat": np.zeros(q.shape, np.int8), "qscale": np.zeros((B, H, nblk), np.float32),
            "khat": np.zeros(k.shape, np.int8), "kscale": np.zeros((B, Hk, nblk), np.float32),
            "kmean": np.zeros((B, Hk, d), np.float32),
        }
    g = (lambda n: _ptr(st[n])) if stages else (lambda n: None)
    rc = lib().orc_attention_sage_blk(C.byref(sh), _ptr(q), _ptr(k), _ptr(v), int(causal),
                                      _ptr(out), g("qhat"), g("qscale"), g("khat"),
                                      g("kscale"), g("kmean"), _threads(threads))
    if rc:
        raise OracleError("attention_sage_blk: bad shape")
    return (out, st) if stages else out


def head_logits(head, hidden, threads=0):
    """engine/mod.rs:781-800 Engine::logits: head (vocab, d) f32, hidden
    (batch, d) or (d,) f32 -> logits (batch, vocab) / (vocab,)."""
    head = np.ascontiguousarray(head, np.float32)
    vocab, d = head.shape
    h = np.ascontiguousarray(hidden, np.float32)
    one = h.ndim == 1
    h2 = h.reshape(-1, d)
    out = np.zeros((h2.shape[0], vocab), np.float32)
    lib().orc_head_logits(_ptr(head), vocab, d, _ptr(h2), h2.shape[0], _ptr(out), _threads(threads))
    return out[0] if one else out


# ---- the transformer trunk (engine/mod.rs:878-945, 763-800) ------------------

def rms_norm_f32(x, w, eps) -> np.ndarray:
    """engine/mod.rs:1152-1160 rms_norm_into (sequential f32 sum of squares)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rms_norm_f32(_ptr(x), _ptr(w), x.size, float(eps), _ptr(out))
    return out


def norm_apply(x, w, eps, serving) -> np.ndarray:
    """engine/mod.rs:837-852 norm_apply: fp32 serving is rms_norm_into as is;
    bf16 serving rounds the operand to bf16 first and the output after."""
    if serving == "fp32":
        return rms_norm_f32(x, w, eps)
    xb = bf16_to_f32(f32_to_bf16(np.asarray(x, np.float32)))
    return bf16_to_f32(f32_to_bf16(rms_norm_f32(xb, w, eps)))


def per_head_norm(v, w, head_dim, eps, serving) -> np.ndarray:
    """engine/mod.rs:854-876 per_head_norm: norm_apply on every head_dim slice
    with one head_dim weight."""
    v = np.asarray(v, np.float32)
    return np.concatenate([norm_apply(v[i:i + head_dim], w, eps, serving)
                           for i in range(0, v.size, head_dim)])


def rope(v, head_dim, pos, theta) -> np.ndarray:
    """engine/mod.rs:1169-1187 rope_rotate (f64 angles, f32 rotation)."""
    v = np.array(v, np.float32)
    lib().orc_rope_rotate(_ptr(v), v.size, int(head_dim), int(pos), float(theta))
    return v


def gqa_attention_scalar(qh, k_cache, v_cache, n_heads, n_kv_heads, head_dim, pos) -> np.ndarray:
    """engine/mod.rs:1073-1116: one query position over the row-major cache
    rows 0..pos (f32 [rows][n_kv_heads * head_dim])."""
    q = np.ascontiguousarray(qh, np.float32)
    kc = np.ascontiguousarray(k_cache[:pos + 1], np.float32)
    vc = np.ascontiguousarray(v_cache[:pos + 1], np.float32)
    out = np.zeros(n_heads * head_dim, np.float32)
    scratch = np.zeros(pos + 1, np.float32)
    lib().orc_gqa_attention_scalar(_ptr(q), _ptr(kc), _ptr(vc), n_heads, n_kv_heads, head_dim, pos,
                                   _ptr(out), _ptr(scratch))
    return out


def swiglu(g, u) -> np.ndarray:
    """engine/mod.rs:930-934: g * u / (1 + exp(-g)) in f32 (exp rounded from
    the f64 value, as libm's correctly rounded expf gives)."""
    g = np.asarray(g, np.float32)
    u = np.asarray(u, np.float32)
    e = np.exp(-g.astype(np.float64)).astype(np.float32)
    return ((g * u).astype(np.float32) / (np.float32(1.0) + e).astype(np.float32)).astype(np.float32)


def block_step(layers, norms, h, pos, k_cache, v_cache, n_heads, n_kv_heads, head_dim, theta, eps,
               serving="fp32", attention="scalar", block=64) -> np.ndarray:
    """engine/mod.rs:886-941, one block at position pos.  layers: the seven
    layer dicts q, k, v, o, gate, up, down (dout, din, r, ub, vt, s1, s2,
    bias); norms: {"input", "post_attention"[, "q_norm", "k_norm"]}; the
    caches are f32 [capacity][n_kv_heads * head_dim], row pos written here.
    serving "fp32" (apply: f64 matvecs) or "bf16" (apply_bf16); attention
    "scalar" (gqa_attention_scalar, the default face) or "sage" (row 0 of the
    padded reference-scheme call, :984-1030, block `block`)."""
    def proj(L, x):
        return factor_apply(serving, L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                            L["bias"], x)

    q_l, k_l, v_l, o_l, g_l, u_l, d_l = layers
    h = np.asarray(h, np.float32)
    x = norm_apply(h, norms["input"], eps, serving)
    q, k, v = proj(q_l, x), proj(k_l, x), proj(v_l, x)
    if "q_norm" in norms and "k_norm" in norms:
        q = per_head_norm(q, norms["q_norm"], head_dim, eps, serving)
        k = per_head_norm(k, norms["k_norm"], head_dim, eps, serving)
    q = rope(q, head_dim, pos, theta)
    k = rope(k, head_dim, pos, theta)
    k_cache[pos] = k
    v_cache[pos] = v
    if attention == "scalar":
        attn = gqa_attention_scalar(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, pos)
    else:
        seq = pos + 1
        qp = np.zeros((1, n_heads, seq, head_dim), np.float32)
        qp[0, :, 0, :] = q.reshape(n_heads, head_dim)
        kp = np.ascontiguousarray(k_cache[:seq].reshape(seq, n_kv_heads, head_dim).transpose(1, 0, 2))[None]
        vp = np.ascontiguousarray(v_cache[:seq].reshape(seq, n_kv_heads, head_dim).transpose(1, 0, 2))[None]
        attn = attention_sage_dev(qp, kp, vp, False, block)[0, :, 0, :].reshape(-1)
    h1 = (proj(o_l, attn) + h).astype(np.float32)
    x2 = norm_apply(h1, norms["post_attention"], eps, serving)
    hid = swiglu(proj(g_l, x2), proj(u_l, x2))
    return (proj(d_l, hid) + h1).astype(np.float32)


def bf16_round(x) -> np.ndarray:
    """f32 values rounded to bf16 (RNE, half 2.7.1 from_f32) and widened back."""
    return bf16_to_f32(f32_to_bf16(np.asarray(x, np.float32)))


def heads_major(rows, n_heads, head_dim) -> np.ndarray:
    """Token rows (n, n_heads * head_dim) -> the attention operand (1, n_heads,
    n, head_dim): head h's slice of row t becomes [0, h, t]
    (KvCache::head_major, engine/mod.rs:1236-1268)."""
    rows = np.asarray(rows, np.float32)
    n = rows.shape[0]
    return np.ascontiguousarray(rows.reshape(n, n_heads, head_dim).transpose(1, 0, 2))[None]


def token_rows(att) -> np.ndarray:
    """The inverse of heads_major: (n_heads, n, dv) -> (n, n_heads * dv)."""
    att = np.asarray(att, np.float32)
    return np.ascontiguousarray(att.transpose(1, 0, 2)).reshape(att.shape[1], -1)


def prefill_qkv(layers, norms, h_rows, k_cache, v_cache, head_dim, theta, eps):
    """The first half of engine/mod.rs:886-921 for every row t of a prefill at
    bf16 serving, position t: input norm, the q/k/v projections (apply_bf16),
    per-head q/k norms when the block has them, RoPE at position t, cache rows
    t written.  Returns the q, k, v rows (n, width) f32."""
    def proj(L, x):
        return factor_apply("bf16", L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                            L["bias"], x)

    q_l, k_l, v_l = layers[:3]
    h_rows = np.asarray(h_rows, np.float32)
    qs, ks, vs = [], [], []
    for t in range(h_rows.shape[0]):
        x = norm_apply(h_rows[t], norms["input"], eps, "bf16")
        q, k, v = proj(q_l, x), proj(k_l, x), proj(v_l, x)
        if "q_norm" in norms and "k_norm" in norms:
            q = per_head_norm(q, norms["q_norm"], head_dim, eps, "bf16")
            k = per_head_norm(k, norms["k_norm"], head_dim, eps, "bf16")
        q, k = rope(q, head_dim, t, theta), rope(k, head_dim, t, theta)
        k_cache[t], v_cache[t] = k, v
        qs.append(q)
        ks.append(k)
        vs.append(v)
    return np.stack(qs), np.stack(ks), np.stack(vs)


def prefill_attention(q_rows, k_rows, v_rows, n_heads, n_kv_heads, head_dim):
    """The prefill's attention (the step of engine/mod.rs:922-925 for every
    row at once): the rows' bf16 q, k, v taken head-major, the causal
    block-scaled SageAttention over the n tokens, the heads back to token rows
    and rounded to bf16 -- the o projection's operand, as the device stores
    it.  Returns (n, n_heads * head_dim) f32 holding bf16 values."""
    qb = f32_to_bf16(heads_major(q_rows, n_heads, head_dim))
    kb = f32_to_bf16(heads_major(k_rows, n_kv_heads, head_dim))
    vb = f32_to_bf16(heads_major(v_rows, n_kv_heads, head_dim))
    att = attention_sage_blk(qb, kb, vb, causal=True)[0]                        # (H, n, hd) f32
    return bf16_round(token_rows(att))


def prefill_mlp(layers, norms, h_rows, att_rows, eps):
    """The second half of engine/mod.rs:922-941 for every row: o projection +
    residual, post-attention norm, gate/up, SwiGLU, down + residual, at bf16
    serving.  Returns the block's output rows."""
    def proj(L, x):
        return factor_apply("bf16", L["dout"], L["din"], L["r"], L["ub"], L["vt"], L["s1"], L["s2"],
                            L["bias"], x)

    o_l, g_l, u_l, d_l = layers[3:]
    h_rows = np.asarray(h_rows, np.float32)
    out = np.zeros_like(h_rows)
    for t in range(h_rows.shape[0]):
        h1 = (proj(o_l, att_rows[t]) + h_rows[t]).astype(np.float32)
        x2 = norm_apply(h1, norms["post_attention"], eps, "bf16")
        hid = swiglu(proj(g_l, x2), proj(u_l, x2))
        out[t] = (proj(d_l, hid) + h1).astype(np.float32)
    return out


def block_prefill(layers, norms, h_rows, k_cache, v_cache, n_heads, n_kv_heads, head_dim, theta, eps):
    """The device block prefill's arithmetic at bf16 serving: every row of
    engine/mod.rs:886-941 at positions 0 .. n - 1 (prefill_qkv), with the
    attention of the n tokens the causal block-scaled SageAttention over their
    bf16 q, k, v (prefill_attention), then the MLP half (prefill_mlp).  The
    reference prefills by running this block token by token
    (engine/mod.rs:1399-1402); the cache rows are the ones block_step writes.
    Returns the output rows; fills cache rows 0 .. n - 1."""
    q, k, v = prefill_qkv(layers, norms, h_rows, k_cache, v_cache, head_dim, theta, eps)
    att = prefill_attention(q, k, v, n_heads, n_kv_heads, head_dim)
    return prefill_mlp(layers, norms, h_rows, att, eps)


class Trunk:
    """Engine::forward_prefill (engine/mod.rs:805-822): per token, the
    embedding row, every block over its KV cache, the final norm and the
    logits (Engine::logits, :788-800).  Built from a model directory (or any
    object with the same fields) at a serving dtype; under bf16 serving the
    remainder tensors are rounded to bf16 (engine/mod.rs:695-706)."""

    def __init__(self, md, serving="fp32", attention="scalar", capacity=None, block=64):
        self.md, self.serving, self.attention, self.block = md, serving, attention, block
        q = bf16_round if serving == "bf16" else \
            (lambda a: np.asarray(a, np.float32))
        self.embedding = q(md.embedding)
        self.head = q(md.head_rows())
        self.final_norm = q(md.final_norm())
        self.blocks = []
        for b in range(md.n_layers):
            layers = [qpk1_layer(s) for s in md.block_layers(b)]
            norms = {k: q(v) for k, v in md.block_norms(b).items()}
            self.blocks.append((layers, norms))
        cap = capacity or 4096
        kv = md.n_kv_heads * md.head_dim
        self.kc = [np.zeros((cap, kv), np.float32) for _ in range(md.n_layers)]
        self.vc = [np.zeros((cap, kv), np.float32) for _ in range(md.n_layers)]
        self.pos = 0

    def reset(self):
        self.pos = 0

    def hidden(self, token: int) -> np.ndarray:
        """engine/mod.rs:878-945 transformer over one token at the next
        position: the final-normed hidden row."""
        md = self.md
        h = self.embedding[int(token)].copy()
        for b, (layers, norms) in enumerate(self.blocks):
            h = block_step(layers, norms, h, self.pos, self.kc[b], self.vc[b], md.n_heads, md.n_kv_heads,
                           md.head_dim, md.rope_theta, md.rms_norm_eps, self.serving, self.attention,
                           self.block)
        self.pos += 1
        return norm_apply(h, self.final_norm, md.rms_norm_eps, self.serving)

    def step(self, token: int) -> np.ndarray:
        """Engine::forward (:802-806): the logits of one token."""
        return head_logits(self.head, self.hidden(token))
