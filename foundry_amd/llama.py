"""Llama decoder with q4 weights on the HIP backend: the caller of the q4 path.

Mirrors the reference's model call sites (src/models/llama/model.rs:92-194,
src/models/llama/attention.rs:72-132, src/models/llama/mlp.rs:49-58) and its
greedy driver (src/generate/mod.rs:45-204):

    h = embed(ids)                                  (q4 gather, tied table)
    for each layer:
        x = rms_norm(h);  q,k,v = x Wq, x Wk, x Wv  (one GEMV/GEMM on [Wq;Wk;Wv])
        q,k = rope(q,k); cache k,v; a = attention(q, cache) Wo
        h = h + a; x = rms_norm(h)
        m = (silu(x Wgate) * (x Wup)) Wdown          (one GEMV/GEMM on [Wgate;Wup])
        h = h + m
    logits = rms_norm(h)[last] Wembed^T;  next = argmax(logits)

Fusions that keep each output row's arithmetic unchanged:
- q/k/v and gate/up weights are concatenated along N (each output row of a
  linear depends only on its own weight row);
- each residual add is fused into the RMSNorm that follows it;
- up to 8 rows (decode), each RMSNorm is formed inside the GEMV that consumes
  it (fh_q4_matmul_rmsnorm, the residual stream alternating between two
  buffers), SiLU*up inside the gate/up GEMV (fh_q4_gate_up_silu), and one
  new token's RoPE and cache write inside attention (fh_decode_attention).

The layer loop itself runs in the library (fh_llama_forward over an
fh_llama_model table built once here). The decode step reads its token id and
position from device memory, so it is captured once as a HIP graph and
replayed for every generated token. Weights
are random-init (SplitMix64-seeded); no checkpoint is read.
"""
from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass, field

import numpy as np

from . import _lib, synth
from .device import HipDevice, HipStorage

GROUP = 64


@dataclass(frozen=True)
class RopeScaling:
    """Llama3RopeScaling (src/models/llama/config.rs:31-36)."""

    factor: float = 32.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_max_position_embeddings: int = 8192


@dataclass(frozen=True)
class LlamaConfig:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_scaling: RopeScaling | None = field(default_factory=RopeScaling)
    max_position_embeddings: int = 131072
    eos_token_id: tuple = ()

    @staticmethod
    def parse(data: bytes) -> "LlamaConfig":
        """LlamaConfig::parse (src/models/llama/config.rs:104-200): a config.json
        of model_type "llama" with heads * head_dim == hidden (head_dim derived
        when absent), heads a multiple of the KV heads, llama3 RoPE scaling or
        none, and tied embeddings; LlamaError of the reference's kind
        otherwise."""
        from .weights import LlamaError

        try:
            f = json.loads(bytes(data).decode("utf-8"))
        except (UnicodeDecodeError, ValueError) as e:
            raise LlamaError("ConfigJson", str(e)) from None

        def req(key, kind):
            if not isinstance(f, dict) or key not in f:
                raise LlamaError("ConfigJson", f"missing {key}")
            v = f[key]
            ok = {"usize": isinstance(v, int) and not isinstance(v, bool) and v >= 0,
                  "f32": isinstance(v, (int, float)) and not isinstance(v, bool),
                  "str": isinstance(v, str), "bool": isinstance(v, bool)}[kind]
            if not ok:
                raise LlamaError("ConfigJson", f"{key}={v!r}")
            return v

        model_type = req("model_type", "str")
        hidden, inter, layers = req("hidden_size", "usize"), req("intermediate_size", "usize"), req("num_hidden_layers", "usize")
        heads, kv = req("num_attention_heads", "usize"), req("num_key_value_heads", "usize")
        eps, theta = req("rms_norm_eps", "f32"), req("rope_theta", "f32")
        max_pos, vocab, tied = req("max_position_embeddings", "usize"), req("vocab_size", "usize"), req("tie_word_embeddings", "bool")
        hd = f.get("head_dim")
        if hd is not None and (not isinstance(hd, int) or isinstance(hd, bool) or hd < 0):
            raise LlamaError("ConfigJson", f"head_dim={hd!r}")
        eos = f.get("eos_token_id", None)
        if isinstance(eos, int) and not isinstance(eos, bool) and 0 <= eos < 2 ** 32:
            eos = (eos,)
        elif isinstance(eos, list) and all(isinstance(e, int) and not isinstance(e, bool) and 0 <= e < 2 ** 32 for e in eos):
            eos = tuple(eos)
        else:
            raise LlamaError("ConfigJson", f"eos_token_id={eos!r}")
        rs = f.get("rope_scaling")
        if rs is not None:
            if not isinstance(rs, dict):
                raise LlamaError("ConfigJson", "rope_scaling")
            for key, kind in (("rope_type", str), ("factor", (int, float)), ("low_freq_factor", (int, float)),
                              ("high_freq_factor", (int, float)), ("original_max_position_embeddings", int)):
                if not isinstance(rs.get(key), kind) or isinstance(rs.get(key), bool):
                    raise LlamaError("ConfigJson", f"rope_scaling.{key}")
        if model_type != "llama":
            raise LlamaError("ModelType", model_type)
        head_dim = hd if hd is not None else (hidden // heads if heads else None)
        if head_dim is None or heads * head_dim != hidden:
            raise LlamaError("HiddenSizeMismatch", f"hidden {hidden}, heads {heads}, head_dim {hd}")
        if kv == 0 or heads % kv != 0:
            raise LlamaError("HeadRatio", f"heads {heads}, kv heads {kv}")
        if rs is not None and rs["rope_type"] != "llama3":
            raise LlamaError("RopeType", rs["rope_type"])
        if not tied:
            raise LlamaError("UntiedEmbeddings")
        f32 = lambda v: float(np.float32(v))
        scaling = None if rs is None else RopeScaling(f32(rs["factor"]), f32(rs["low_freq_factor"]),
                                                      f32(rs["high_freq_factor"]),
                                                      int(rs["original_max_position_embeddings"]))
        return LlamaConfig(layers, hidden, heads, kv, head_dim, inter, vocab, f32(eps), f32(theta), scaling, max_pos,
                           eos)

    @staticmethod
    def open(directory) -> "LlamaConfig":
        """LlamaConfig::open: <directory>/config.json, at most 1 MiB."""
        from .weights import LlamaError

        path = os.path.join(directory, "config.json")
        try:
            if os.path.getsize(path) > 1024 * 1024:
                raise LlamaError("ConfigTooLarge", path)
            with open(path, "rb") as fh:
                data = fh.read()
        except OSError as e:
            raise LlamaError("ConfigRead", str(e)) from None
        return LlamaConfig.parse(data)

    @staticmethod
    def llama_3_2_3b() -> "LlamaConfig":
        return LlamaConfig(28, 3072, 24, 8, 128, 8192, 128256)

    @staticmethod
    def llama_3_1_8b() -> "LlamaConfig":
        return LlamaConfig(32, 4096, 32, 8, 128, 14336, 128256)

    @property
    def qkv_rows(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


def inv_freq(cfg: LlamaConfig) -> np.ndarray:
    """src/models/llama/rotary_emb.rs:135-186, in float32."""
    d = cfg.head_dim
    theta = np.float32(cfg.rope_theta)
    out = []
    for i in range(0, d, 2):
        f = np.float32(1.0) / np.power(theta, np.float32(i) / np.float32(d), dtype=np.float32)
        sc = cfg.rope_scaling
        if sc is not None:
            ctx = np.float32(sc.original_max_position_embeddings)
            low, high = np.float32(sc.low_freq_factor), np.float32(sc.high_freq_factor)
            factor = np.float32(sc.factor)
            wl_low, wl_high = ctx / low, ctx / high
            wl = np.float32(2 * np.pi) / f
            fs = f / factor if wl > wl_low else f
            smooth = (ctx / wl - low) / (high - low)
            if wl_high <= wl <= wl_low:
                fs = (np.float32(1) - smooth) * fs / factor + smooth * fs
            f = np.float32(fs)
        out.append(f)
    return np.array(out, dtype=np.float32)


def rope_tables(cfg: LlamaConfig, length: int):
    """cos/sin tables [length, head_dim] in bf16 (src/models/llama/rotary_emb.rs:87-131):
    angle = position * inv_freq in float32, duplicated over both halves."""
    f = inv_freq(cfg)
    f2 = np.concatenate([f, f])
    pos = np.arange(length, dtype=np.float32)[:, None]
    ang = (pos * f2[None, :]).astype(np.float32)
    return synth.bf16_rne(np.cos(ang).astype(np.float32)), synth.bf16_rne(np.sin(ang).astype(np.float32))


class _Q4:
    """A q4 weight triplet on the device. With ``interleave`` (k a multiple
    of 128) also fh_q4_interleave's copy of its scales and biases, and with
    ``tile`` (n a multiple of 16, 32 for ``silu_pairs``) fh_q4_tile's copy of
    its words, both read by the batched decode GEMVs instead of the triplet
    (the same values: results do not change)."""

    def __init__(self, dev: HipDevice, wq: np.ndarray, s: np.ndarray, b: np.ndarray, interleave: bool = True,
                 tile: bool = False, silu_pairs: bool = False):
        self.n, self.k = wq.shape[0], wq.shape[1] * 8
        self.wq = dev.storage_from_bytes(np.ascontiguousarray(wq).tobytes())
        self.s = dev.storage_from_bytes(np.ascontiguousarray(s).tobytes())
        self.b = dev.storage_from_bytes(np.ascontiguousarray(b).tobytes())
        self.sb = self.wt = None
        if interleave and self.k % (2 * GROUP) == 0 and self.n > 0:
            self.sb = dev.empty(self.n * (self.k // GROUP) * 4)
            _lib.call("fh_q4_interleave", dev.handle, ctypes.c_void_p(self.s.ptr), ctypes.c_void_p(self.b.ptr),
                      self.n, self.k, GROUP, ctypes.c_void_p(self.sb.ptr))
            if tile and self.n % (32 if silu_pairs else 16) == 0:
                self.wt = dev.empty(self.n * self.k // 2)
                _lib.call("fh_q4_tile", dev.handle, ctypes.c_void_p(self.wq.ptr), self.n, self.k, GROUP,
                          int(silu_pairs), ctypes.c_void_p(self.wt.ptr))


def layer_weights(cfg: LlamaConfig, seed: int, layer: int, centre: float = 8.0):
    """Host-side random-init q4 weights of one layer: dict of (wq, s, b)
    triplets and bf16 norm weights. Layer l's packed words are layer 0's xor a
    per-layer constant (uniform nibbles stay uniform), so building a
    28-layer model costs one layer's draws. ``centre`` sets the biases
    (synth.q4_weights): 8 is the task's distribution, 7.5 zero-mean weights."""
    key = np.uint32((0x9E3779B9 * (layer + 1)) & 0xFFFFFFFF)
    out = {}
    for name, (n, k, s_off) in {
        "qkv": (cfg.qkv_rows, cfg.hidden, 1),
        "o": (cfg.hidden, cfg.n_heads * cfg.head_dim, 2),
        "gate_up": (2 * cfg.ffn, cfg.hidden, 3),
        "down": (cfg.hidden, cfg.ffn, 4),
    }.items():
        wq, s, b = _cached_q4(seed * 16 + s_off, n, k, centre)
        out[name] = (wq ^ key if layer else wq, s, b)
    for name, s_off in (("input_norm", 5), ("post_norm", 6)):
        out[name] = _norm_weight(seed * 16 + s_off + 97 * layer, cfg.hidden)
    return out


_CACHE: dict = {}


def _cached_q4(seed: int, n: int, k: int, centre: float = 8.0):
    key = (seed, n, k, centre)
    if key not in _CACHE:
        _CACHE[key] = synth.q4_weights(seed, n, k, GROUP, centre)
    return _CACHE[key]


def _norm_weight(seed: int, n: int) -> np.ndarray:
    z = synth.bf16_to_f32(synth.bf16_normal(seed, (n,))).astype(np.float64)
    return synth.bf16_rne((1.0 + 0.1 * z).astype(np.float32))


def embed_weights(cfg: LlamaConfig, seed: int, centre: float = 8.0):
    return _cached_q4(seed * 16 + 7, cfg.vocab, cfg.hidden, centre)


def final_norm_weight(cfg: LlamaConfig, seed: int):
    return _norm_weight(seed * 16 + 8, cfg.hidden)


class Q4Llama:
    """Random-init q4 Llama on one device. It runs `batch` sequences of equal
    length (batch_dims, src/generate/mod.rs:207-225), each with a static KV
    cache of `max_len` positions per layer, laid out [batch, n_kv, max_len,
    head_dim] (StaticCache, src/nn/kv_cache.rs:13-39). `max_tokens` bounds the
    tokens of one sequence in one forward."""

    def __init__(self, dev: HipDevice, cfg: LlamaConfig, seed: int | None, max_len: int, max_tokens: int,
                 batch: int = 1, weights=None, centre: float = 8.0, interleave: bool = True):
        """Weights are random-init from `seed` (biases centred at -centre * s,
        see layer_weights), or read from `weights` (a
        foundry_amd.weights.Weights of q4 triplets; see from_checkpoint).
        `interleave`: also keep each weight's scales and biases interleaved
        (fh_q4_interleave, 1/8 more weight memory) and, for batch 2..8, its
        words tiled in the batched GEMV's task order (fh_q4_tile, twice the
        weight memory) for the batched decode GEMVs; the results are the same
        either way."""
        self.dev, self.cfg, self.max_len = dev, cfg, max_len
        if max_len > cfg.max_position_embeddings:
            raise ValueError("max_len exceeds max_position_embeddings")
        if not 1 <= batch <= 65535:
            raise ValueError(f"batch {batch} must be in 1..65535")
        self.batch = int(batch)
        self.max_tokens = max(1, max_tokens)
        self.seq_bytes = cfg.n_kv_heads * max_len * cfg.head_dim * 2  # one sequence's cache, per layer
        if weights is not None:
            from .weights import llama_final_norm, llama_q4_embed, llama_q4_layer
            src_embed, src_layer, src_norm = (lambda: llama_q4_embed(weights, cfg),
                                              lambda l: llama_q4_layer(weights, cfg, l),
                                              lambda: llama_final_norm(weights, cfg))
        else:
            src_embed, src_layer, src_norm = (lambda: embed_weights(cfg, seed, centre),
                                              lambda l: layer_weights(cfg, seed, l, centre),
                                              lambda: final_norm_weight(cfg, seed))
        tile = interleave and 2 <= self.batch <= 8  # the batched GEMVs read tiled words
        self.embed = _Q4(dev, *src_embed(), interleave=interleave, tile=tile)
        self.layers = []
        for layer in range(cfg.n_layers):
            w = src_layer(layer)
            self.layers.append({
                "qkv": _Q4(dev, *w["qkv"], interleave=interleave, tile=tile),
                "o": _Q4(dev, *w["o"], interleave=interleave, tile=tile),
                "gate_up": _Q4(dev, *w["gate_up"], interleave=interleave, tile=tile, silu_pairs=True),
                "down": _Q4(dev, *w["down"], interleave=interleave, tile=tile),
                "input_norm": dev.storage_from_bytes(w["input_norm"].tobytes()),
                "post_norm": dev.storage_from_bytes(w["post_norm"].tobytes()),
                "k_cache": dev.zeros(self.batch * self.seq_bytes),
                "v_cache": dev.zeros(self.batch * self.seq_bytes),
            })
        self.final_norm = dev.storage_from_bytes(np.ascontiguousarray(src_norm()).tobytes())
        cos, sin = rope_tables(cfg, max_len)
        self.cos = dev.storage_from_bytes(cos.tobytes())
        self.sin = dev.storage_from_bytes(sin.tobytes())
        self.scale = float(np.float32(1.0) / np.sqrt(np.float32(cfg.head_dim), dtype=np.float32))
        t, c, bt = self.max_tokens, cfg, self.batch
        r = bt * t  # rows of one forward
        self.buf = {
            "h": dev.empty(r * c.hidden * 2),
            "h2": dev.empty(r * c.hidden * 2),
            "x": dev.empty(r * c.hidden * 2),
            "qkv": dev.empty(r * c.qkv_rows * 2),
            "q": dev.empty(r * c.n_heads * c.head_dim * 2),
            "attn": dev.empty(r * c.n_heads * c.head_dim * 2),
            "o": dev.empty(r * c.hidden * 2),
            "gu": dev.empty(r * 2 * c.ffn * 2),
            "act": dev.empty(r * c.ffn * 2),
            "logits": dev.empty(bt * c.vocab * 2),
            "ids": dev.empty(r * 4),
            "positions": dev.empty(r * 4),
            "next": dev.zeros(bt * 4),
            "pos1": dev.zeros(bt * 4),
        }
        # prefill attention runs one sequence at a time, reusing one workspace
        self.attn_ws_bytes = _lib.attention_workspace_bytes(t, c.n_heads, c.n_kv_heads, c.head_dim, max_len)
        self.attn_ws = dev.zeros(self.attn_ws_bytes)
        self.dec_ws_bytes = _lib.decode_attention_workspace_bytes(bt, c.n_heads, c.n_kv_heads, c.head_dim, max_len)
        self.dec_ws = dev.zeros(self.dec_ws_bytes)
        self.seq_len = 0
        self._model = self._native_model()

    def _native_model(self) -> _lib.LlamaModel:
        """The fh_llama_model that fh_llama_forward runs: the config, every
        layer's device operands and the forward's buffers (device pointers)."""
        c, b = self.cfg, self.buf

        def q4(w: _Q4) -> _lib.Q4Weight:
            return _lib.Q4Weight(w.wq.ptr, w.s.ptr, w.b.ptr, w.n, w.k, w.sb.ptr if w.sb is not None else None,
                                 w.wt.ptr if w.wt is not None else None)

        self._layer_table = (_lib.LlamaLayer * len(self.layers))(*[
            _lib.LlamaLayer(q4(L["qkv"]), q4(L["o"]), q4(L["gate_up"]), q4(L["down"]), L["input_norm"].ptr,
                            L["post_norm"].ptr, L["k_cache"].ptr, L["v_cache"].ptr) for L in self.layers])
        m = _lib.LlamaModel(n_layers=c.n_layers, hidden=c.hidden, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads,
                            head_dim=c.head_dim, ffn=c.ffn, vocab=c.vocab, batch=self.batch, max_len=self.max_len,
                            max_tokens=self.max_tokens, rms_norm_eps=c.rms_norm_eps, scale=self.scale,
                            layers=self._layer_table, embed=q4(self.embed), final_norm=self.final_norm.ptr,
                            cos_tab=self.cos.ptr, sin_tab=self.sin.ptr, attn_workspace=self.attn_ws.ptr,
                            attn_workspace_bytes=self.attn_ws_bytes, decode_workspace=self.dec_ws.ptr,
                            decode_workspace_bytes=self.dec_ws_bytes)
        for name, key in (("h", "h"), ("h2", "h2"), ("x", "x"), ("qkv", "qkv"), ("q", "q"), ("attn", "attn"),
                          ("o", "o"), ("gate_up", "gu"), ("act", "act"), ("logits", "logits")):
            setattr(m, name, b[key].ptr)
        return m

    @classmethod
    def from_checkpoint(cls, dev: HipDevice, directory, max_len: int, max_tokens: int, batch: int = 1) -> "Q4Llama":
        """A q4 checkpoint directory: config.json (LlamaConfig::open) and
        model.safetensors or an index with shards, holding q4 triplets
        ({name}.weight U32, .scales / .biases BF16) for the embedding (tied
        LM head) and every projection, and BF16 norm weights
        (src/models/llama/model.rs:130-160 names)."""
        from .weights import Weights
        cfg = LlamaConfig.open(directory)
        return cls(dev, cfg, None, max_len, max_tokens, batch, weights=Weights.open(directory))

    def _p(self, st: HipStorage, byte_offset: int = 0):
        return ctypes.c_void_p(st.ptr + byte_offset)

    def _forward(self, seq_tokens: int, ids: HipStorage, positions: HipStorage):
        """One forward over `seq_tokens` rows of every sequence (rows ordered
        sequence-major), issued by fh_llama_forward: embedding, every layer,
        the LM head of each sequence's last row and its argmax, which is left
        in buf['next'] (src/models/llama/model.rs:92-121)."""
        _lib.call("fh_llama_forward", self.dev.handle, ctypes.addressof(self._model), seq_tokens, self._p(ids),
                  self._p(positions), self._p(self.buf["next"]))

    def _upload(self, st: HipStorage, arr: np.ndarray):
        _lib.call("fh_upload", self.dev.handle, self._p(st), arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)

    # ---- prefill and decode ----
    def step(self, ids: np.ndarray, past: int) -> None:
        """One forward of ids [batch, T] at positions past..past+T-1 of every
        sequence (Decoder::step, src/generate/mod.rs:150-204): caches those
        positions and leaves each sequence's greedy next id on the device
        (buf['next']) and past + T in buf['pos1']."""
        ids = np.ascontiguousarray(np.atleast_2d(ids), dtype=np.uint32)
        rows, t = ids.shape
        if rows != self.batch:
            raise ValueError(f"{rows} sequences given to a model built for batch {self.batch}")
        if t == 0 or t > self.max_tokens or past < 0 or past + t > self.max_len:
            raise ValueError(f"{t} tokens at position {past} do not fit (max_tokens {self.max_tokens}, "
                             f"max_len {self.max_len})")
        self._upload(self.buf["ids"], ids)
        self._upload(self.buf["positions"], np.tile(np.arange(past, past + t, dtype=np.uint32), rows))
        self._forward(t, self.buf["ids"], self.buf["positions"])
        self._upload(self.buf["pos1"], np.full(rows, past + t, dtype=np.uint32))
        self.seq_len = past + t

    def prefill(self, prompt: np.ndarray, past: int = 0) -> None:
        """Runs the prompt ([T] for one sequence, else [batch, T]) from
        position `past`; the first generated ids are left on the device."""
        self.step(prompt, past)

    def capture_decode(self, log: HipStorage, capacity: int):
        """Captures one decode step: each sequence's token in buf['next'] at
        position buf['pos1'] -> its next token, logged at log[seq, pos -
        seq_len + 1] (index 0 is the prefill's token), then position + 1."""
        d = self.dev.handle
        self.dev.capture_begin()
        try:
            self._forward(1, self.buf["next"], self.buf["pos1"])
            _lib.call("fh_append_token_advance", d, self._p(self.buf["next"]), self.batch, self._p(log),
                      self._p(self.buf["pos1"]), self.seq_len - 1, capacity, 1)
        except Exception:
            self.dev.capture_end()
            raise
        return self.dev.capture_end()

    def generate(self, prompt: np.ndarray, new_tokens: int, depth: np.ndarray | None = None):
        """Greedy generation (src/generate/mod.rs:45-90): returns the new ids
        ([new_tokens] for a 1-D prompt, else [batch, new_tokens]; the first
        is the prefill's argmax). `depth` ([batch, D]) is run first at
        positions 0..D-1, as the bench's depth rows (src/bench/mod.rs:
        250-262)."""
        single = np.ndim(prompt) == 1
        past = 0
        if depth is not None and np.size(depth):
            depth = np.atleast_2d(depth)
            for s in range(0, depth.shape[1], self.max_tokens):
                self.step(depth[:, s:s + self.max_tokens], s)
            past = depth.shape[1]
        self.step(prompt, past)
        if self.seq_len + new_tokens - 1 > self.max_len:
            raise ValueError("generation would run past the KV cache")
        first = np.empty(self.batch, dtype=np.uint32)
        _lib.call("fh_download", self.dev.handle, first.ctypes.data_as(ctypes.c_void_p), self._p(self.buf["next"]),
                  first.nbytes)
        out = np.zeros((self.batch, max(new_tokens, 0)), dtype=np.uint32)
        if new_tokens > 1:
            log = self.dev.zeros(4 * self.batch * new_tokens)
            graph = self.capture_decode(log, new_tokens)
            for _ in range(new_tokens - 1):
                graph.launch()
            _lib.call("fh_download", self.dev.handle, out.ctypes.data_as(ctypes.c_void_p), self._p(log), out.nbytes)
        if new_tokens > 0:
            out[:, 0] = first
        return out[0] if single else out

    def next_tokens(self) -> np.ndarray:
        """Each sequence's greedy next id (reads back, so it synchronises)."""
        out = np.empty(self.batch, dtype=np.uint32)
        _lib.call("fh_download", self.dev.handle, out.ctypes.data_as(ctypes.c_void_p), self._p(self.buf["next"]),
                  out.nbytes)
        return out

    def eager_step(self) -> None:
        """One decode step launched op by op: every sequence's token in
        buf['next'] at position buf['pos1'] -> its next token; position + 1."""
        self._forward(1, self.buf["next"], self.buf["pos1"])
        _lib.call("fh_advance_positions", self.dev.handle, self._p(self.buf["pos1"]), self.batch, 1)

    def capture_step(self):
        """The decode step (eager_step) captured once as a HIP graph; replay
        it with .launch()."""
        if getattr(self, "_step_graph", None) is None:
            self.dev.capture_begin()
            try:
                self.eager_step()
            except Exception:
                self.dev.capture_end()
                raise
            self._step_graph = self.dev.capture_end()
        return self._step_graph

    def weight_bytes(self) -> int:
        """Device bytes of the weights (packed words, scales, biases, norms)."""
        q4 = [self.embed] + [L[k] for L in self.layers for k in ("qkv", "o", "gate_up", "down")]
        n = sum(w.wq.nbytes + w.s.nbytes + w.b.nbytes for w in q4)
        return n + sum(L[k].nbytes for L in self.layers for k in ("input_norm", "post_norm")) + self.final_norm.nbytes

    def parameter_count(self) -> int:
        """Logical parameters: every q4 weight element (not its scales and
        biases) and every norm weight; the LM head shares the embedding."""
        q4 = [self.embed] + [L[k] for L in self.layers for k in ("qkv", "o", "gate_up", "down")]
        return sum(w.n * w.k for w in q4) + (2 * len(self.layers) + 1) * self.cfg.hidden

    def logits(self) -> np.ndarray:
        """Last computed logits (bf16 bits) of each sequence's final position:
        [vocab] for batch 1, else [batch, vocab]."""
        out = np.empty((self.batch, self.cfg.vocab), dtype=np.uint16)
        _lib.call("fh_download", self.dev.handle, out.ctypes.data_as(ctypes.c_void_p), self._p(self.buf["logits"]),
                  out.nbytes)
        return out[0] if self.batch == 1 else out
