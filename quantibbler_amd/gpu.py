"""Device face: GpuContext, FactorLayer, FactorSet, AttentionShape.

Mirrors crates/quantibbler-kernels/src/gpu.rs (GpuContext::init / init_at /
packed_matvec, gpu_available) and gpu_attention.rs (AttentionShape,
attention_sage), plus the device-resident factor linear of the engine's
PackedLayer (crates/quantibbler-server/src/engine/mod.rs:313-481).

Host-buffer methods take and return NumPy arrays (copy in, launch, copy
out, like the reference).  ``*_dev`` methods take device pointers (ints, or
objects with ``data_ptr()`` such as torch tensors) and a stream handle, and
return without waiting.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import AttnShape, check

_DTYPES = {"float64": (_lib.QBK_F64, np.float64), "float32": (_lib.QBK_F32, np.float32),
           "bfloat16": (_lib.QBK_BF16, np.uint16)}


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    raise TypeError(f"cannot take a pointer of {type(x)!r}")


def _nbytes(x):
    """Bytes behind a buffer given as a tensor or an array (None for a raw
    address, whose size the caller vouches for)."""
    if hasattr(x, "element_size") and hasattr(x, "numel"):
        return int(x.element_size() * x.numel())
    if isinstance(x, np.ndarray):
        return int(x.nbytes)
    return None


def _stream(s):
    if s is None:
        return None
    if isinstance(s, int):
        return s
    if hasattr(s, "cuda_stream"):
        return s.cuda_stream
    raise TypeError(f"cannot take a stream handle of {type(s)!r}")


def gpu_available() -> bool:
    """gpu.rs:187-189."""
    return bool(_lib.load().qbk_gpu_available())


@dataclass(frozen=True)
class AttentionShape:
    """gpu_attention.rs:402-411."""
    batch: int
    n_heads: int
    n_kv_heads: int
    seq_q: int
    seq_kv: int
    head_dim: int
    val_dim: int

    def c(self) -> AttnShape:
        return AttnShape(self.batch, self.n_heads, self.n_kv_heads, self.seq_q, self.seq_kv,
                         self.head_dim, self.val_dim)


class GpuContext:
    """gpu.rs:76-185: a live context on one gfx950 device (fail-closed init)."""

    def __init__(self, device_index: int = 0):
        lib = _lib.load()
        h = C.c_void_p()
        check(lib.qbk_ctx_create(int(device_index), C.byref(h)))
        self._h = h
        self.device_index = int(device_index)

    @classmethod
    def init(cls) -> "GpuContext":
        return cls(0)

    @classmethod
    def init_at(cls, device_index: int) -> "GpuContext":
        return cls(device_index)

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            _lib.load().qbk_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- packed products (gpu.rs:116-185, dispatch.rs:81-109) -------------

    def packed_matvec(self, packed, n_rows: int, n_bits: int, vec, dtype: str = "float64"):
        code, npdt = _DTYPES[dtype]
        p = np.ascontiguousarray(packed, dtype=np.uint8).ravel()
        v = np.ascontiguousarray(vec, dtype=npdt).ravel()
        # the library refuses f64 shapes past the reference device face's u32
        # index ceiling (gpu.rs:127-137) before any device use or write to out,
        # so such a call is made without an output buffer
        big = dtype == "float64" and max(p.size, int(n_rows)) > 0xFFFFFFFF
        out = None if big else np.zeros(n_rows, dtype=npdt)
        check(_lib.load().qbk_packed_matvec(self._h, code, _ptr(p), p.size, n_rows, n_bits,
                                            _ptr(v), v.size, _ptr(out)))
        return out

    def packed_matmul(self, packed, n_rows: int, n_bits: int, mat, n_cols: int,
                      dtype: str = "float64"):
        code, npdt = _DTYPES[dtype]
        p = np.ascontiguousarray(packed, dtype=np.uint8).ravel()
        m = np.ascontiguousarray(mat, dtype=npdt).ravel()
        k = m.size // max(n_bits, 1)
        out = np.zeros(n_rows * k, dtype=npdt)
        check(_lib.load().qbk_packed_matmul(self._h, code, _ptr(p), p.size, n_rows, n_bits,
                                            _ptr(m), m.size, n_cols, _ptr(out)))
        return out.reshape(n_rows, k)

    # ---- attention (gpu_attention.rs:451-756) -----------------------------

    def attention(self, shape: AttentionShape, query, key, value, causal: bool):
        """gpu_attention.rs:451-570 GpuContext::attention: exact f32
        attention, Q unscaled, GQA, bottom-right causal; (B*H*Sq*dv,) f32."""
        q = np.ascontiguousarray(query, dtype=np.float32).ravel()
        k = np.ascontiguousarray(key, dtype=np.float32).ravel()
        v = np.ascontiguousarray(value, dtype=np.float32).ravel()
        out = np.zeros(shape.batch * shape.n_heads * shape.seq_q * shape.val_dim, np.float32)
        sh = shape.c()
        check(_lib.load().qbk_attention(self._h, C.byref(sh), _ptr(q), q.size, _ptr(k), k.size, _ptr(v),
                                        v.size, int(bool(causal)), _ptr(out)))
        return out

    def attention_dev(self, shape: AttentionShape, q, k, v, causal: bool, out, stream=None):
        sh = shape.c()
        check(_lib.load().qbk_attention_dev(self._h, C.byref(sh), _ptr(q), _ptr(k), _ptr(v),
                                            int(bool(causal)), _ptr(out), _stream(stream)))


    def attention_sage(self, shape: AttentionShape, query, key, value, causal: bool,
                       block_size: int):
        q = np.ascontiguousarray(query, dtype=np.float32).ravel()
        k = np.ascontiguousarray(key, dtype=np.float32).ravel()
        v = np.ascontiguousarray(value, dtype=np.float32).ravel()
        out = np.zeros(shape.batch * shape.n_heads * shape.seq_q * shape.val_dim, np.float32)
        sh = shape.c()
        check(_lib.load().qbk_attention_sage(self._h, C.byref(sh), _ptr(q), q.size, _ptr(k),
                                             k.size, _ptr(v), v.size, int(bool(causal)),
                                             int(block_size), _ptr(out)))
        return out

    def attention_sage_dev(self, shape: AttentionShape, q, k, v, causal: bool, block_size: int,
                           out, stream=None):
        sh = shape.c()
        check(_lib.load().qbk_attention_sage_dev(self._h, C.byref(sh), _ptr(q), _ptr(k), _ptr(v),
                                                 int(bool(causal)), int(block_size), _ptr(out),
                                                 _stream(stream)))

    # ---- one decode step over a KV cache (engine/mod.rs:984-1030) ----------

    def attention_sage_decode(self, shape: AttentionShape, query, key_cache, value_cache,
                              block_size: int):
        """Row 0 of the reference's padded decode call (gqa_attention_sage:
        the step's query in row 0 of a (pos + 1)-row problem, causal=False),
        computed alone.  query (n_heads, d); key_cache (seq_kv, n_kv_heads,
        d) and value_cache (seq_kv, n_kv_heads, dv) as the cache holds them
        (row-major); shape: batch 1, seq_q 1, seq_kv = pos + 1.  Returns
        (n_heads, dv) f32."""
        q = np.ascontiguousarray(query, dtype=np.float32).ravel()
        k = np.ascontiguousarray(key_cache, dtype=np.float32).ravel()
        v = np.ascontiguousarray(value_cache, dtype=np.float32).ravel()
        out = np.zeros(shape.n_heads * shape.val_dim, np.float32)
        sh = shape.c()
        check(_lib.load().qbk_attention_sage_decode(self._h, C.byref(sh), _ptr(q), q.size, _ptr(k),
                                                    k.size, _ptr(v), v.size, int(block_size),
                                                    _ptr(out), out.size))
        return out.reshape(shape.n_heads, shape.val_dim)

    def sage_decode_workspace_size(self, shape: AttentionShape, block_size: int) -> int:
        sh = shape.c()
        return int(_lib.load().qbk_sage_decode_workspace_size(C.byref(sh), int(block_size)))

    def attention_sage_decode_dev(self, shape: AttentionShape, q, key_cache, value_cache,
                                  block_size: int, out, workspace, workspace_size: int,
                                  stream=None):
        sh = shape.c()
        check(_lib.load().qbk_attention_sage_decode_dev(self._h, C.byref(sh), _ptr(q),
                                                        _ptr(key_cache), _ptr(value_cache),
                                                        int(block_size), _ptr(out),
                                                        _ptr(workspace), int(workspace_size),
                                                        _stream(stream)))

    def attention_sage_decode_step_dev(self, shape: AttentionShape, q, key_cache, value_cache,
                                       block_size: int, out, state, state_size: int, capacity: int,
                                       cached_tokens: int, stream=None):
        sh = shape.c()
        check(_lib.load().qbk_attention_sage_decode_step_dev(
            self._h, C.byref(sh), _ptr(q), _ptr(key_cache), _ptr(value_cache), int(block_size),
            _ptr(out), _ptr(state), int(state_size), int(capacity), int(cached_tokens),
            _stream(stream)))

    def sage_blk_workspace_size(self, shape: AttentionShape) -> int:
        sh = shape.c()
        return int(_lib.load().qbk_sage_blk_workspace_size(C.byref(sh)))

    def attention_sage_blk_dev(self, shape: AttentionShape, q, k, v, causal: bool, out,
                               workspace, workspace_size: int, stream=None):
        sh = shape.c()
        check(_lib.load().qbk_attention_sage_blk_dev(self._h, C.byref(sh), _ptr(q), _ptr(k),
                                                     _ptr(v), int(bool(causal)), _ptr(out),
                                                     _ptr(workspace), int(workspace_size),
                                                     _stream(stream)))

    def sage_blk_quantize_dev(self, shape: AttentionShape, q, k, v, qhat, qscale, khat, kscale,
                              kmean, vh, stream=None):
        sh = shape.c()
        check(_lib.load().qbk_sage_blk_quantize_dev(self._h, C.byref(sh), _ptr(q), _ptr(k),
                                                    _ptr(v), _ptr(qhat), _ptr(qscale),
                                                    _ptr(khat), _ptr(kscale), _ptr(kmean),
                                                    _ptr(vh), _stream(stream)))


def embed(ctx: GpuContext, table, vocab: int, d_model: int, tokens, out, stream=None):
    """engine/mod.rs:768-778 Engine::embed: host token ids (validated with the
    reference's text) -> f32 rows of the device table into ``out``."""
    t = np.ascontiguousarray(tokens, np.int32).ravel()
    check(_lib.load().qbk_embed(ctx.handle, _ptr(table), int(vocab), int(d_model), _ptr(t), t.size, _ptr(out),
                                _stream(stream)))


def embed_dev(ctx: GpuContext, table, vocab: int, d_model: int, tokens, n: int, out, stream=None):
    """Device token ids (int32); an out-of-range id yields a NaN row."""
    check(_lib.load().qbk_embed_dev(ctx.handle, _ptr(table), int(vocab), int(d_model), _ptr(tokens), int(n),
                                    _ptr(out), _stream(stream)))


def rms_norm_dev(ctx: GpuContext, x, rows: int, d: int, w, eps: float, out, stream=None, serving: str = "bf16"):
    """The final norm (engine/mod.rs:943) per row at the serving dtype:
    "bf16" (operand and output rounded to bf16) or "fp32" (as is)."""
    fn = _lib.load().qbk_rms_norm_f32_dev if serving == "fp32" else _lib.load().qbk_rms_norm_dev
    check(fn(ctx.handle, _ptr(x), int(rows), int(d), _ptr(w), float(eps), _ptr(out), _stream(stream)))


def advance_positions_dev(ctx: GpuContext, pos, n: int, stream=None):
    """pos[i] += 1 for the n device uint32 positions of a greedy loop."""
    check(_lib.load().qbk_positions_advance_dev(ctx.handle, _ptr(pos), int(n), _stream(stream)))


def argmax_dev(ctx: GpuContext, logits, rows: int, vocab: int, out, stream=None):
    """sampler.rs:4-15 greedy, per row (int32 ids into ``out``)."""
    check(_lib.load().qbk_argmax_dev(ctx.handle, _ptr(logits), int(rows), int(vocab), _ptr(out),
                                     _stream(stream)))


class SageDecodeState:
    """A decode loop's attention state for one layer (engine/mod.rs:984-1030
    gqa_attention_sage, called once per generated token over a growing
    KvCache): a device buffer, supplied by the caller, laid out for a cache
    of ``capacity`` tokens, and the number of cache rows whose codes it holds.
    Each step re-quantises only the key blocks from the last complete one on;
    the output is bit-identical to a fresh call.  ``reset()`` after the
    cache's earlier rows change (a new sequence)."""

    def __init__(self, ctx: GpuContext, n_heads: int, n_kv_heads: int, head_dim: int,
                 val_dim: int, capacity: int, block_size: int, state):
        self.ctx = ctx
        self.n_heads, self.n_kv_heads = int(n_heads), int(n_kv_heads)
        self.head_dim, self.val_dim = int(head_dim), int(val_dim)
        self.capacity, self.block_size = int(capacity), int(block_size)
        self.state = state
        need = self.size(ctx, n_heads, n_kv_heads, head_dim, val_dim, capacity, block_size)
        have = _nbytes(state)
        if have is not None and have < need:
            raise _lib.KernelError(f"decode state of {have} bytes is smaller than the {need} a "
                                   f"capacity of {capacity} tokens needs")
        self.state_size = have if have is not None else need
        self.tokens = 0

    @staticmethod
    def size(ctx: GpuContext, n_heads, n_kv_heads, head_dim, val_dim, capacity, block_size) -> int:
        """Bytes of device memory a state for ``capacity`` tokens needs."""
        shape = AttentionShape(1, n_heads, n_kv_heads, 1, capacity, head_dim, val_dim)
        return ctx.sage_decode_workspace_size(shape, block_size)

    def reset(self):
        self.tokens = 0

    def step(self, q, key_cache, value_cache, seq_kv: int, out, stream=None):
        """Attention of the step's query ``q`` (n_heads, head_dim) over the
        first ``seq_kv`` rows of the row-major caches into ``out``
        (n_heads, val_dim); a cache shorter than the last step's starts over."""
        seq_kv = int(seq_kv)
        cached = self.tokens if self.tokens <= seq_kv else 0
        shape = AttentionShape(1, self.n_heads, self.n_kv_heads, 1, seq_kv, self.head_dim,
                               self.val_dim)
        self.ctx.attention_sage_decode_step_dev(shape, q, key_cache, value_cache,
                                                self.block_size, out, self.state,
                                                self.state_size, self.capacity, cached, stream)
        self.tokens = seq_kv


class DecoderBlock:
    """One decoder block of the server's transformer at one position
    (engine/mod.rs:878-945; bf16 serving, the sage decode attention on a
    kept state): norm -> q/k/v -> [per-head q/k norms] -> RoPE -> cache
    append -> attention -> o + residual -> norm -> gate/up -> SwiGLU ->
    down + residual, on the device.  ``layers`` are the seven FactorLayers
    q, k, v, o, gate, up, down (kept alive here); ``q_norm``/``k_norm`` are
    optional head_dim weights; the block owns its KV cache of ``capacity``
    rows."""

    def __init__(self, ctx: GpuContext, layers, input_norm, post_norm, n_heads: int,
                 n_kv_heads: int, head_dim: int, rope_theta: float, rms_norm_eps: float,
                 capacity: int, block_size: int = 64, q_norm=None, k_norm=None, n_seqs: int = 1):
        if len(layers) != 7:
            raise _lib.KernelError("a decoder block takes 7 layers: q, k, v, o, gate, up, down")
        self.ctx = ctx
        self.layers = list(layers)
        self.d_model = self.layers[3].dout
        arr = (C.c_void_p * 7)(*[L.handle for L in self.layers])
        w_in = np.ascontiguousarray(input_norm, np.float32).ravel()
        w_post = np.ascontiguousarray(post_norm, np.float32).ravel()
        wq = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32).ravel()
        wk = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32).ravel()
        qk_len = 0 if wq is None else wq.size
        if wq is not None and wk is not None and wk.size != wq.size:
            raise _lib.KernelError(f"decoder block: q/k norm weights of {wq.size} and {wk.size} floats differ")
        out = C.c_void_p()
        check(_lib.load().qbk_block_create_seqs(ctx.handle, arr, _ptr(w_in), w_in.size, _ptr(w_post),
                                                w_post.size, _ptr(wq), _ptr(wk), qk_len, int(n_heads),
                                                int(n_kv_heads), int(head_dim), float(rope_theta),
                                                float(rms_norm_eps), int(capacity), int(block_size), int(n_seqs),
                                                C.byref(out)))
        self._h = out
        self.capacity = int(capacity)
        self.n_seqs = int(n_seqs)
        self.face = "sage"
        self.serving = "bf16"

    def decode_dev(self, h, pos: int, stream=None):
        """h: device f32 [d_model] (a contiguous torch tensor, or a raw device
        address the caller vouches for), replaced by the block's output at
        position pos."""
        if hasattr(h, "is_cuda"):
            if not h.is_cuda or str(h.dtype) != "torch.float32" or not h.is_contiguous() \
                    or h.numel() != self.d_model:
                raise _lib.KernelError(
                    f"decoder block input must be a contiguous float32 device tensor of {self.d_model} "
                    f"values; got {h.dtype} of {h.numel()} on {h.device}")
        elif not isinstance(h, int):
            raise _lib.KernelError("decoder block input must be a device tensor or a device address")
        check(_lib.load().qbk_block_decode_dev(self.ctx.handle, self._h, _ptr(h), int(pos),
                                               _stream(stream)))

    def prefill_workspace_size(self, n_tokens: int) -> int:
        return int(_lib.load().qbk_block_prefill_workspace_size(self._h, int(n_tokens)))

    def prefill_dev(self, h, n_tokens: int, workspace, workspace_size: int, stream=None):
        """A new sequence's first n_tokens positions in one pass: h device f32
        [n_tokens][d_model] rows, replaced by the block's outputs; decoding
        continues at position n_tokens."""
        if hasattr(h, "is_cuda"):
            if not h.is_cuda or str(h.dtype) != "torch.float32" or not h.is_contiguous() \
                    or h.numel() != self.d_model * int(n_tokens):
                raise _lib.KernelError(
                    f"prefill input must be a contiguous float32 device tensor of {n_tokens} x {self.d_model} "
                    f"values; got {h.dtype} of {h.numel()} on {h.device}")
        check(_lib.load().qbk_block_prefill_dev(self.ctx.handle, self._h, _ptr(h), int(n_tokens), _ptr(workspace),
                                                int(workspace_size), _stream(stream)))

    def prefill_seq_dev(self, seq: int, h, n_tokens: int, workspace, workspace_size: int, stream=None):
        """prefill_dev for sequence ``seq`` of a block holding several."""
        self._check_rows(h, int(n_tokens), "prefill input")
        check(_lib.load().qbk_block_prefill_seq_dev(self.ctx.handle, self._h, int(seq), _ptr(h), int(n_tokens),
                                                    _ptr(workspace), int(workspace_size), _stream(stream)))

    def decode_batch_workspace_size(self, n: int) -> int:
        return int(_lib.load().qbk_block_decode_batch_workspace_size(self._h, int(n)))

    def decode_batch_dev(self, h, positions, workspace, workspace_size: int, stream=None):
        """One position of each of sequences 0 .. n - 1: h device f32
        [n][d_model], row i sequence i's token, replaced by the block's
        outputs; positions[i] as decode_dev's pos for sequence i."""
        pos = np.ascontiguousarray(positions, np.uint64).ravel()
        n = pos.size
        self._check_rows(h, n, "batched decode input")
        check(_lib.load().qbk_block_decode_batch_dev(self.ctx.handle, self._h, _ptr(h),
                                                     _ptr(pos), n, _ptr(workspace),
                                                     int(workspace_size), _stream(stream)))

    def decode_pos_dev(self, h, pos, stream=None):
        """decode_dev at the position the device uint32 ``pos`` holds when
        the step runs (a HIP graph of the step serves every position); the
        kept attention state must be stepped through pos - 1.  The block's
        host record of positions is left as it was (set_positions)."""
        self._check_rows(h, 1, "decoder block input")
        self._check_pos(pos, 1)
        check(_lib.load().qbk_block_decode_pos_dev(self.ctx.handle, self._h, _ptr(h), _ptr(pos),
                                                   _stream(stream)))

    def decode_batch_pos_dev(self, h, pos, n: int, workspace, workspace_size: int, stream=None):
        """decode_batch_dev with the n positions in the device uint32 tensor
        ``pos``, read when the step runs."""
        self._check_rows(h, int(n), "batched decode input")
        self._check_pos(pos, int(n))
        check(_lib.load().qbk_block_decode_batch_pos_dev(self.ctx.handle, self._h, _ptr(h), _ptr(pos), int(n),
                                                         _ptr(workspace), int(workspace_size), _stream(stream)))

    def set_positions(self, positions):
        """The host record after device-position steps: sequence i holds
        positions[i] positions, its attention state stepped through them."""
        p = np.ascontiguousarray(positions, np.uint64).ravel()
        check(_lib.load().qbk_block_set_positions(self._h, _ptr(p), p.size))

    def set_filled(self, rows):
        """Sequence i holds rows[i] cache rows written through cache_ptrs();
        its attention state is rebuilt from them on the next eager step."""
        p = np.ascontiguousarray(rows, np.uint64).ravel()
        check(_lib.load().qbk_block_set_filled(self._h, _ptr(p), p.size))

    @staticmethod
    def _check_pos(pos, n: int):
        if hasattr(pos, "is_cuda"):
            if not pos.is_cuda or str(pos.dtype) not in ("torch.int32", "torch.uint32") \
                    or not pos.is_contiguous() or pos.numel() < n:
                raise _lib.KernelError(f"positions must be a contiguous 32-bit device tensor of at least {n} "
                                       f"entries; got {pos.dtype} of {pos.numel()} on {pos.device}")
        elif not isinstance(pos, int):
            raise _lib.KernelError("positions must be a device tensor or a device address")

    def _check_rows(self, h, n: int, what: str):
        if hasattr(h, "is_cuda"):
            if not h.is_cuda or str(h.dtype) != "torch.float32" or not h.is_contiguous() \
                    or h.numel() != self.d_model * n:
                raise _lib.KernelError(
                    f"{what} must be a contiguous float32 device tensor of {n} x {self.d_model} "
                    f"values; got {h.dtype} of {h.numel()} on {h.device}")
        elif not isinstance(h, int):
            raise _lib.KernelError(f"{what} must be a device tensor or a device address")

    ATTENTION_FACES = {"sage": 0, "exact": 1}

    def set_attention_face(self, face: str):
        """The attention face of the block's steps (engine/mod.rs:953-968):
        "sage" (the default: the reference-scheme sage decode attention on a
        kept state) or "exact" (f32 attention over the cached rows, the
        gpu:tiled face; one sequence at host positions -- decode_dev and
        prefill_dev, the latter token by token)."""
        if face not in self.ATTENTION_FACES:
            raise _lib.KernelError(f"attention face must be one of {sorted(self.ATTENTION_FACES)}, got {face!r}")
        check(_lib.load().qbk_block_set_attention_face(self._h, self.ATTENTION_FACES[face]))
        self.face = face

    SERVING = {"fp32": 1, "bf16": 2}

    def set_serving(self, serving: str):
        """The block's serving dtype (engine/mod.rs ServingDtype): "bf16"
        (the default) or "fp32" -- apply's f64 products and f32 norms, one
        sequence at host positions (decode_dev, prefill_dev token by
        token).  The first "fp32" call forms the layers' row bitplanes."""
        if serving not in self.SERVING:
            raise _lib.KernelError(f"serving must be one of {sorted(self.SERVING)}, got {serving!r}")
        check(_lib.load().qbk_block_set_serving(self.ctx.handle, self._h, self.SERVING[serving]))
        self.serving = serving

    def reset(self):
        check(_lib.load().qbk_block_reset(self._h))

    def cache_ptrs(self):
        k, v = C.c_void_p(), C.c_void_p()
        check(_lib.load().qbk_block_cache(self._h, C.byref(k), C.byref(v)))
        return k.value, v.value

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h:
            _lib.load().qbk_block_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LmHead:
    """Device-resident language-model head (engine/mod.rs:781-800
    Engine::logits): logits[v] = sum_t hidden[t] * head[v][t], one f32 sum
    per vocabulary row in t order -- bit-identical to the reference's loop.
    Stored transposed, as bf16 when every element is a bf16 value."""

    def __init__(self, ctx: GpuContext, handle):
        self._ctx = ctx
        self._h = handle
        v, d, b = C.c_size_t(), C.c_size_t(), C.c_int()
        check(_lib.load().qbk_head_info(handle, C.byref(v), C.byref(d), C.byref(b)))
        self.vocab, self.d_model, self.bf16 = v.value, d.value, bool(b.value)

    @classmethod
    def from_rows(cls, ctx: GpuContext, head) -> "LmHead":
        h = np.ascontiguousarray(head, dtype=np.float32)
        vocab, d = h.shape
        out = C.c_void_p()
        check(_lib.load().qbk_head_create(ctx.handle, _ptr(h), h.size, vocab, d, C.byref(out)))
        return cls(ctx, out)

    @classmethod
    def from_rows_dev(cls, ctx: GpuContext, head_dev, vocab: int, d_model: int) -> "LmHead":
        out = C.c_void_p()
        check(_lib.load().qbk_head_create_dev(ctx.handle, _ptr(head_dev), int(vocab), int(d_model),
                                              C.byref(out)))
        return cls(ctx, out)

    @property
    def handle(self):
        return self._h

    def logits(self, hidden) -> np.ndarray:
        h = np.ascontiguousarray(hidden, dtype=np.float32)
        rows = h.size // max(self.d_model, 1)
        out = np.zeros(rows * self.vocab, np.float32)
        check(_lib.load().qbk_head_logits(self._ctx.handle, self._h, _ptr(h), h.size, _ptr(out), out.size))
        return out.reshape(self.vocab) if h.ndim == 1 else out.reshape(rows, self.vocab)

    def logits_dev(self, hidden, batch: int, logits, stream=None):
        check(_lib.load().qbk_head_logits_dev(self._ctx.handle, self._h, _ptr(hidden), int(batch),
                                              _ptr(logits), _stream(stream)))

    def close(self):
        if self._h:
            _lib.load().qbk_head_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class FactorLayer:
    """Device-resident binary factor linear (engine/mod.rs:313-481 PackedLayer)."""

    def __init__(self, ctx: GpuContext, handle):
        self.ctx = ctx
        self._h = handle
        d = [C.c_size_t() for _ in range(3)]
        check(_lib.load().qbk_factor_dims(handle, *[C.byref(x) for x in d]))
        self.dout, self.din, self.r = (x.value for x in d)

    @classmethod
    def from_qpk1(cls, ctx: GpuContext, stream: bytes) -> "FactorLayer":
        b = np.frombuffer(bytes(stream), dtype=np.uint8)
        h = C.c_void_p()
        check(_lib.load().qbk_factor_from_qpk1(ctx.handle, _ptr(b), b.size, C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_rows(cls, ctx: GpuContext, dout: int, din: int, r: int, ub_rows, vb_t_rows, s1, s2,
                  bias=None) -> "FactorLayer":
        ub = np.ascontiguousarray(ub_rows, np.uint8)
        vt = np.ascontiguousarray(vb_t_rows, np.uint8)
        a1 = np.ascontiguousarray(s1, np.float32)
        a2 = np.ascontiguousarray(s2, np.float32)
        bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
        if ub.size != dout * ((r + 7) // 8) or vt.size != r * ((din + 7) // 8):
            raise _lib.KernelError("bitplane length mismatch after repack")
        if a1.size != dout or a2.size != din or (bb is not None and bb.size != dout):
            raise _lib.KernelError(
                f"scale/bias lengths ({a1.size}, {a2.size}, {None if bb is None else bb.size}) "
                f"do not match (dout={dout}, din={din})")
        h = C.c_void_p()
        check(_lib.load().qbk_factor_from_rows(ctx.handle, dout, din, r, _ptr(ub), _ptr(vt),
                                               _ptr(a1), _ptr(a2), _ptr(bb), C.byref(h)))
        return cls(ctx, h)

    @property
    def handle(self):
        return self._h

    def workspace_size(self, batch: int) -> int:
        return int(_lib.load().qbk_factor_workspace_size(self._h, batch))

    def linear_dev(self, x, batch: int, y, y_dtype: str, workspace, workspace_size: int,
                   stream=None):
        code = _DTYPES[y_dtype][0]
        check(_lib.load().qbk_factor_linear_dev(self.ctx.handle, self._h, _ptr(x), batch,
                                                _ptr(y), code, _ptr(workspace),
                                                int(workspace_size), _stream(stream)))

    def linear_noalloc_dev(self, x, batch: int, y, y_dtype: str, stream=None):
        """linear_dev without a workspace: the library's per-GPU scratch
        array (QBK_NOALLOC_SCRATCH_BYTES); allocates nothing.  Calls that
        overlap on one GPU race."""
        code = _DTYPES[y_dtype][0]
        check(_lib.load().qbk_factor_linear_noalloc_dev(self.ctx.handle, self._h, _ptr(x), int(batch),
                                                        _ptr(y), code, _stream(stream)))

    def apply(self, x, serving: str = "bfloat16") -> np.ndarray:
        """PackedLayer::apply ("float32": f64 matvecs) / apply_bf16 ("bfloat16")."""
        code = _DTYPES[serving][0]
        xx = np.ascontiguousarray(x, np.float32)
        batch = xx.size // self.din
        if batch * self.din != xx.size:
            raise _lib.KernelError(f"layer expects input dim {self.din}, got {xx.shape[-1]}")
        y = np.zeros((batch, self.dout), np.float32)
        check(_lib.load().qbk_factor_apply(self.ctx.handle, self._h, code, _ptr(xx), batch,
                                           _ptr(y)))
        return y if xx.ndim > 1 else y[0]

    def close(self):
        if getattr(self, "_h", None):
            _lib.load().qbk_factor_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class FactorSet:
    """Layers (any shapes) decoded together at batch 1 in three launches;
    x and y are the concatenations of the layers' x_i and y_i."""

    def __init__(self, ctx: GpuContext, layers):
        self.ctx = ctx
        self.layers = list(layers)
        arr = (C.c_void_p * len(self.layers))(*[l.handle.value for l in self.layers])
        h = C.c_void_p()
        check(_lib.load().qbk_factor_set_create(ctx.handle, arr, len(self.layers), C.byref(h)))
        self._h = h

    def workspace_size(self) -> int:
        return int(_lib.load().qbk_factor_set_workspace_size(self._h))

    def decode_dev(self, x, y, workspace, workspace_size: int, stream=None):
        check(_lib.load().qbk_factor_set_decode_dev(self.ctx.handle, self._h, _ptr(x), _ptr(y),
                                                    _ptr(workspace), int(workspace_size),
                                                    _stream(stream)))

    def workspace_size_batch(self, n: int) -> int:
        return int(_lib.load().qbk_factor_set_workspace_size_batch(self._h, int(n)))

    def decode_batch_dev(self, n: int, x, y, workspace, workspace_size: int, stream=None):
        """Every layer at a batch of n tokens (1 .. 32): x bf16 [layer][n][din],
        y bf16 [layer][n][dout], device pointers or tensors."""
        check(_lib.load().qbk_factor_set_decode_batch_dev(self.ctx.handle, self._h, int(n), _ptr(x), _ptr(y),
                                                          _ptr(workspace), int(workspace_size), _stream(stream)))

    def shared_workspace_size(self, n: int) -> int:
        return int(_lib.load().qbk_factor_set_shared_workspace_size(self._h, int(n)))

    def shared_dev(self, n: int, x, y, workspace, workspace_size: int, stream=None):
        """Layers that read the same input (q/k/v, gate/up) at a batch of n
        tokens (1 .. 64) on the prefill GEMM: x bf16 [n][din], y bf16
        [layer][n][dout]."""
        check(_lib.load().qbk_factor_set_shared_dev(self.ctx.handle, self._h, int(n), _ptr(x), _ptr(y),
                                                    _ptr(workspace), int(workspace_size), _stream(stream)))

    def stage_dev(self, stage: int, x, y, workspace, workspace_size: int, stream=None):
        check(_lib.load().qbk_factor_set_stage_dev(self.ctx.handle, self._h, int(stage), _ptr(x),
                                                   _ptr(y), _ptr(workspace), int(workspace_size),
                                                   _stream(stream)))

    def close(self):
        if getattr(self, "_h", None):
            _lib.load().qbk_factor_set_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
