"""Model directory reader: the host half of the reference's directory load
(crates/quantibbler-qpk1/src/loader.rs:172-320 `load`, composed by
crates/quantibbler-server/src/model/mod.rs:582-597 and
engine/mod.rs:639-760 `ModelWeights::from_layers`), for the files a
quantized model directory holds:

* ``config.toml`` -- geometry (vocab_size, d_model, n_layers, n_heads,
  n_kv_heads, head_dim, rms_norm_eps, rope_theta), the norm inventory
  ``norm_slots`` and ``weight_tying``;
* ``manifest.toml`` -- the layer names, ``[layer_files]`` (name -> qpk1 path)
  and ``[sidecar]`` (embedding, lm_head, norms, optional dtype f32|bf16);
* the qpk1 layer streams (parsed and uploaded by ``qbk_factor_from_qpk1``)
  and the raw little-endian remainder tensors.

The norm sidecar is laid out by inventory (engine/mod.rs:517-560
BlockRefs::resolve): per block, the declared slots in order -- ``input``,
``post_attention``, ``post_feedforward`` are d_model floats, ``q_norm`` and
``k_norm`` head_dim floats -- then the final norm's d_model floats.

Only what the fixtures and the hot path use is read; the blob format and the
reference's long list of directory refusals are out of scope.  Errors raise
``ModelError`` naming the file.
"""
from __future__ import annotations

import ast
import os
import re
from dataclasses import dataclass, field

import numpy as np


class ModelError(ValueError):
    """A model directory that cannot be read (the reference's load error)."""


def read_toml(path: str) -> dict:
    """The TOML subset the reference's model files use: comments, [tables],
    bare or double-quoted keys, strings, numbers, booleans and (multi-line)
    arrays of those."""
    out: dict = {}
    table = out
    pending = ""
    try:
        with open(path, encoding="utf-8") as f:
            lines = f.read().splitlines()
    except OSError as e:
        raise ModelError(f"{path}: {e}") from None
    for raw in lines:
        line = _strip_comment(raw).strip()
        if not line and not pending:
            continue
        if pending:
            pending += " " + line
            if pending.count("[") > pending.count("]"):
                continue
            line, pending = pending, ""
        m = re.fullmatch(r"\[\s*([A-Za-z0-9_.\-]+)\s*\]", line)
        if m:
            table = out.setdefault(m.group(1), {})
            continue
        m = re.fullmatch(r'("(?:[^"\\]|\\.)*"|[A-Za-z0-9_\-]+)\s*=\s*(.*)', line)
        if not m:
            raise ModelError(f"{path}: cannot read line {raw!r}")
        key, val = m.group(1), m.group(2)
        if val.count("[") > val.count("]"):
            pending = line
            continue
        if key.startswith('"'):
            key = ast.literal_eval(key)
        table[key] = _value(path, val)
    if pending:
        raise ModelError(f"{path}: unterminated array")
    return out


def _strip_comment(line: str) -> str:
    in_str = False
    for i, ch in enumerate(line):
        if ch == '"' and (i == 0 or line[i - 1] != "\\"):
            in_str = not in_str
        elif ch == "#" and not in_str:
            return line[:i]
    return line


def _value(path, text):
    t = text.strip()
    if t in ("true", "false"):
        return t == "true"
    try:
        return ast.literal_eval(t)
    except (ValueError, SyntaxError):
        raise ModelError(f"{path}: cannot read value {text!r}") from None


_SLOT_WIDTH = {"input": "d", "post_attention": "d", "post_feedforward": "d", "q_norm": "h", "k_norm": "h"}
_DTYPES = {"f32": np.float32, "bf16": np.uint16}


def _remainder(path: str, n: int, dtype: str) -> np.ndarray:
    """A raw little-endian remainder tensor of n values at the declared dtype,
    widened to f32 (bf16 widens exactly)."""
    try:
        raw = np.fromfile(path, dtype="<u2" if dtype == "bf16" else "<f4")
    except OSError as e:
        raise ModelError(f"{path}: {e}") from None
    if raw.size != n:
        raise ModelError(f"{path}: holds {raw.size} {dtype} values; expected {n}")
    if dtype == "bf16":
        return (raw.astype(np.uint32) << 16).view(np.float32)
    return raw.astype(np.float32)


@dataclass
class ModelDir:
    """A model directory read into host memory (f32 remainder tensors, qpk1
    streams by layer name)."""
    path: str
    vocab_size: int
    d_model: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    norm_slots: list
    remainder_dtype: str
    layer_names: list
    streams: dict = field(repr=False)
    embedding: np.ndarray = field(repr=False)
    lm_head: np.ndarray | None = field(repr=False)
    norms: np.ndarray = field(repr=False)

    @classmethod
    def load(cls, path: str) -> "ModelDir":
        cfg = read_toml(os.path.join(path, "config.toml"))
        man = read_toml(os.path.join(path, "manifest.toml"))
        need = ["vocab_size", "d_model", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                "rms_norm_eps", "rope_theta", "norm_slots"]
        for k in need:
            if k not in cfg:
                raise ModelError(f"{path}/config.toml: missing {k}")
        slots = list(cfg["norm_slots"])
        for s in slots:
            if s not in _SLOT_WIDTH:
                raise ModelError(f"{path}/config.toml: unknown norm slot {s!r}")
        side = man.get("sidecar", {})
        dtype = side.get("dtype", "f32")
        if dtype not in _DTYPES:
            raise ModelError(f"{path}/manifest.toml: unknown sidecar dtype {dtype!r}")
        d, h, v, n = int(cfg["d_model"]), int(cfg["head_dim"]), int(cfg["vocab_size"]), int(cfg["n_layers"])
        per_block = sum(d if _SLOT_WIDTH[s] == "d" else h for s in slots)
        files = man.get("layer_files", {})
        names = list(man.get("layers", []))
        streams = {}
        for name in names:
            if name not in files:
                raise ModelError(f"{path}/manifest.toml: layer {name!r} has no [layer_files] entry")
            fp = os.path.join(path, files[name])
            try:
                with open(fp, "rb") as f:
                    streams[name] = f.read()
            except OSError as e:
                raise ModelError(f"{fp}: {e}") from None
        emb = _remainder(os.path.join(path, side.get("embedding", "e1.f32.bin")), v * d, dtype)
        head = None
        if "lm_head" in side and side["lm_head"] != side.get("embedding"):
            head = _remainder(os.path.join(path, side["lm_head"]), v * d, dtype)
        norms = _remainder(os.path.join(path, side.get("norms", "norms.f32.bin")), per_block * n + d, dtype)
        return cls(path=path, vocab_size=v, d_model=d, n_layers=n, n_heads=int(cfg["n_heads"]),
                   n_kv_heads=int(cfg["n_kv_heads"]), head_dim=h, rms_norm_eps=float(cfg["rms_norm_eps"]),
                   rope_theta=float(cfg["rope_theta"]), norm_slots=slots, remainder_dtype=dtype,
                   layer_names=names, streams=streams, embedding=emb.reshape(v, d),
                   lm_head=None if head is None else head.reshape(v, d), norms=norms)

    def head_rows(self) -> np.ndarray:
        """The lm_head rows, or the embedding when tied (engine/mod.rs:788)."""
        return self.embedding if self.lm_head is None else self.lm_head

    def block_norms(self, b: int) -> dict:
        """Block b's norm weights by slot name (engine/mod.rs:517-560)."""
        d, h = self.d_model, self.head_dim
        per_block = sum(d if _SLOT_WIDTH[s] == "d" else h for s in self.norm_slots)
        at = b * per_block
        out = {}
        for s in self.norm_slots:
            w = d if _SLOT_WIDTH[s] == "d" else h
            out[s] = self.norms[at:at + w]
            at += w
        return out

    def final_norm(self) -> np.ndarray:
        return self.norms[-self.d_model:]

    def block_layers(self, b: int) -> list:
        """Block b's seven qpk1 streams in the order q, k, v, o, gate, up,
        down (engine/mod.rs:517-531: names layers.{b}.inner.*)."""
        out = []
        for suffix in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                       "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            name = f"layers.{b}.inner.{suffix}"
            if name not in self.streams:
                raise ModelError(f"block {b}: missing packed layer {name!r}")
            out.append(self.streams[name])
        return out


def _bf16_values(a) -> np.ndarray:
    """f32 values rounded to their bf16 values (round to nearest even; NaN
    kept), as engine/mod.rs:695-706 holds the remainder tensors under bf16
    serving."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32)
    return (r << 16).view(np.float32)


class DeviceModel:
    """The transformer trunk on the device at bf16 serving (Engine::forward,
    engine/mod.rs:802-806, and forward_prefill's per-token loop, :811-822):
    embedding row -> every DecoderBlock over its KV cache -> final norm ->
    lm_head logits, all device-resident.  ``attention`` picks every block's
    face once, as the engine does at load (engine/mod.rs:953-968): "sage"
    (the sage decode attention; prefill on the block-scaled SageAttention)
    or "exact" (f32 attention over the cache, one sequence, prefill token by
    token).  ``serving`` is the engine's serving dtype: "bf16" (remainder
    tensors rounded to bf16, the GEMV / GEMM projections) or "fp32" (the
    tensors as stored, apply's f64 products, f32 norms; one sequence, prefill
    token by token).  Built from a ModelDir; torch supplies the device
    buffers (plumbing only -- every step runs in libqbk)."""

    def __init__(self, ctx, md: ModelDir, capacity: int, block_size: int = 64, n_seqs: int = 1,
                 attention: str = "sage", serving: str = "bf16"):
        import torch

        from .gpu import DecoderBlock, FactorLayer, LmHead

        self.ctx, self.md, self.capacity, self.n_seqs = ctx, md, int(capacity), int(n_seqs)
        if serving not in ("bf16", "fp32"):
            raise ValueError(f"serving must be 'bf16' or 'fp32', got {serving!r}")
        self.serving = serving
        # bf16 serving rounds the remainder tensors to bf16 (engine/mod.rs:695-706)
        rnd = _bf16_values if serving == "bf16" else (lambda a: np.ascontiguousarray(a, np.float32))
        dev = torch.device("cuda")
        self.layers, self.blocks = [], []
        for b in range(md.n_layers):
            layers = [FactorLayer.from_qpk1(ctx, s) for s in md.block_layers(b)]
            self.layers.append(layers)
            norms = {k: rnd(v) for k, v in md.block_norms(b).items()}
            self.blocks.append(DecoderBlock(ctx, layers, norms["input"], norms["post_attention"], md.n_heads,
                                            md.n_kv_heads, md.head_dim, md.rope_theta, md.rms_norm_eps,
                                            capacity, block_size, norms.get("q_norm"), norms.get("k_norm"),
                                            n_seqs=self.n_seqs))
            self.blocks[-1].set_attention_face(attention)
            if serving == "fp32":
                self.blocks[-1].set_serving("fp32")
        self.attention = attention
        self.embedding = torch.from_numpy(rnd(md.embedding)).to(dev)
        self.final_norm = torch.from_numpy(rnd(md.final_norm())).to(dev)
        self.head = LmHead.from_rows(ctx, rnd(md.head_rows()))
        self.h = torch.empty(md.d_model, dtype=torch.float32, device=dev)
        self.hn = torch.empty(md.d_model, dtype=torch.float32, device=dev)
        self.logits = torch.empty(md.vocab_size, dtype=torch.float32, device=dev)
        self.pos = 0                        # sequence 0's, the one step() serves
        self.positions = [0] * self.n_seqs  # every sequence's
        self._batch = {}                    # n -> (h, hn, logits, workspace) of step_batch

    def reset(self):
        for b in self.blocks:
            b.reset()
        self.pos = 0
        self.positions = [0] * self.n_seqs

    def prefill(self, tokens, stream=None, seq: int = 0):
        """forward_prefill (engine/mod.rs:811-822) of a new sequence (held as
        sequence ``seq``) in one pass per block: the tokens' embedding rows
        through every block's prefill (batched projections, causal
        block-scaled SageAttention), then the final norm and logits of the
        last position -- the logits a token-at-a-time prefill ends with.
        Returns them (a device tensor, overwritten by the next call);
        decoding continues with step() (sequence 0) or step_batch()."""
        import torch

        from .gpu import embed, rms_norm_dev

        md = self.md
        ids = [int(t) for t in tokens]
        n = len(ids)
        h = torch.empty((n, md.d_model), dtype=torch.float32, device="cuda")
        embed(self.ctx, self.embedding, md.vocab_size, md.d_model, ids, h, stream)
        need = max(b.prefill_workspace_size(n) for b in self.blocks)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        for b in self.blocks:
            b.prefill_seq_dev(int(seq), h, n, ws, need, stream)
        rms_norm_dev(self.ctx, h[n - 1], 1, md.d_model, self.final_norm, md.rms_norm_eps, self.hn, stream,
                     self.serving)
        self.head.logits_dev(self.hn, 1, self.logits, stream)
        self.positions[int(seq)] = n
        if int(seq) == 0:
            self.pos = n
        return self.logits

    def step_batch(self, tokens, stream=None):
        """One position of each of sequences 0 .. n - 1 (the batched decode of
        engine/mod.rs:1377-1476): ``tokens`` n host ids, or a device int32
        tensor of n ids (a greedy loop's argmax output, fed back without a
        host round trip).  Returns the logits [n][vocab] (a device tensor,
        overwritten by the next call of the same n)."""
        import torch

        from .gpu import embed, embed_dev, rms_norm_dev

        md = self.md
        dev_ids = hasattr(tokens, "is_cuda")
        n = int(tokens.numel()) if dev_ids else len(tokens)
        if n == 0 or n > self.n_seqs:
            raise ValueError(f"a batch of {n} sequences on a model holding {self.n_seqs}")
        if n not in self._batch:
            wn = max(b.decode_batch_workspace_size(n) for b in self.blocks)
            self._batch[n] = (torch.empty((n, md.d_model), dtype=torch.float32, device="cuda"),
                              torch.empty((n, md.d_model), dtype=torch.float32, device="cuda"),
                              torch.empty((n, md.vocab_size), dtype=torch.float32, device="cuda"),
                              torch.empty(wn, dtype=torch.uint8, device="cuda"), wn)
        h, hn, logits, ws, wn = self._batch[n]
        if dev_ids:
            embed_dev(self.ctx, self.embedding, md.vocab_size, md.d_model, tokens, n, h, stream)
        else:
            embed(self.ctx, self.embedding, md.vocab_size, md.d_model, [int(t) for t in tokens], h, stream)
        pos = self.positions[:n]
        for b in self.blocks:
            b.decode_batch_dev(h, pos, ws, wn, stream)
        rms_norm_dev(self.ctx, h, n, md.d_model, self.final_norm, md.rms_norm_eps, hn, stream)
        self.head.logits_dev(hn, n, logits, stream)
        for i in range(n):
            self.positions[i] += 1
        self.pos = self.positions[0]
        return logits

    def step(self, token: int, stream=None):
        """The next position's logits (a device tensor, overwritten by the
        next step) for a host token id."""
        from .gpu import embed, rms_norm_dev

        md = self.md
        embed(self.ctx, self.embedding, md.vocab_size, md.d_model, [int(token)], self.h, stream)
        for b in self.blocks:
            b.decode_dev(self.h, self.pos, stream)
        rms_norm_dev(self.ctx, self.h, 1, md.d_model, self.final_norm, md.rms_norm_eps, self.hn, stream,
                     self.serving)
        self.head.logits_dev(self.hn, 1, self.logits, stream)
        self.pos += 1
        self.positions[0] = self.pos
        return self.logits

    def close(self):
        for b in self.blocks:
            b.close()
        self.head.close()
        for layers in self.layers:
            for L in layers:
                L.close()
