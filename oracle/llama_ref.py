"""CPU restatement of the reference's Llama forward pass: TEST INFRASTRUCTURE ONLY.

Used by tests/ and bench.py's agreement check as the checker of the HIP
decoder (foundry_amd/llama.py). It follows the reference's op sequence and its
bf16 rounding points (every reference tensor op rounds its output to the
tensor dtype, bf16):

- RmsNorm (src/nn/norm.rs:32-50): fp32 sum of squares, scale =
  reciprocal(sqrt(ss * (1/dim) + eps)), y = RNE(RNE(x * scale) * w).
- Linear (src/nn/linear.rs:22-35 -> matmul_tiled): fp32 accumulation of
  x . w, RNE output. (numpy's sgemm sums in a different order than
  matmul_tiled's sequential k; within fp32 accumulation error.) w is the
  weight value the q4 path is specified to consume: a call of at most
  GEMV_MAX_ROWS rows (the decode GEMV) dequantises in registers to the fp32
  s*q + b; a longer call (the prefill GEMM) feeds bf16 matrix cores with
  dequantised tiles, i.e. the materialised bf16 weight RNE(s*q + b). `rows`
  is the row count of the linear call the model makes (batch x tokens).
- RoPE (src/models/llama/rotary_emb.rs:62-85): rot = cat(-x2, x1),
  RNE(RNE(x*cos) + RNE(rot*sin)); tables RNE(cos/sin(pos * inv_freq)) with
  the llama3 frequency scaling (:135-186).
- SDPA (src/nn/attention.rs:23-60): scores RNE(q.k), fp32 scale + causal
  mask, fp32 softmax, RNE probabilities, RNE(p . v).
- Silu * up (src/nn/activation.rs:19-28, src/models/llama/mlp.rs:49-58):
  RNE(RNE(g / (exp(-g) + 1)) * u).
- residual adds RNE(a + b); argmax with ties to the lowest index
  (src/metal/kernels/reduce.metal:42-78).
- generation comparison (src/eval/generation.rs:132-176).

Weights are inputs (the same seeded q4 triplets the GPU model uses).
Pinned by tests/test_llama_ref.py: the reference's own tests of inv_freq,
angles, top-k order, argmax ties and compare_generation, and closed forms for
RmsNorm, SiLU and SDPA.
"""
from __future__ import annotations

import numpy as np

# fh_q4_matmul runs the GEMV up to this many rows and the GEMM above.
GEMV_MAX_ROWS = 8


def rne(x) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even), returned as float32 values."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    r = (((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    nan = np.isnan(f)
    if nan.any():
        r[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint32) << 16
    return r.view(np.float32)


def from_bf16(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequant_f32(wq, s, b, group: int = 64) -> np.ndarray:
    """w = f32(s) * q + f32(b) (one rounding; s*q is exact)."""
    n, kw = wq.shape
    q = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))[None, None, :]) & 0xF).reshape(n, kw * 8)
    sf = np.repeat(from_bf16(s), group, axis=1)
    bf = np.repeat(from_bf16(b), group, axis=1)
    return (sf * q.astype(np.float32)).astype(np.float32) + bf


def inv_freq(head_dim, theta, scaling) -> np.ndarray:
    out = []
    for i in range(0, head_dim, 2):
        f = np.float32(1.0) / np.power(np.float32(theta), np.float32(i) / np.float32(head_dim), dtype=np.float32)
        if scaling is not None:
            factor, low, high, orig = (np.float32(scaling[0]), np.float32(scaling[1]), np.float32(scaling[2]),
                                       np.float32(scaling[3]))
            wl = np.float32(2 * np.pi) / f
            fs = f / factor if wl > orig / low else f
            smooth = (orig / wl - low) / (high - low)
            if orig / high <= wl <= orig / low:
                fs = (np.float32(1) - smooth) * fs / factor + smooth * fs
            f = np.float32(fs)
        out.append(f)
    return np.array(out, dtype=np.float32)


def angles(freqs, length) -> np.ndarray:
    """[length, 2 * len(freqs)]: position * frequency, the frequencies repeated
    for both halves (src/models/llama/rotary_emb.rs:87-133)."""
    f = np.asarray(freqs, dtype=np.float32)
    return (np.arange(length, dtype=np.float32)[:, None] * np.concatenate([f, f])[None, :]).astype(np.float32)


def rope_tables(head_dim, theta, scaling, length):
    ang = angles(inv_freq(head_dim, theta, scaling), length)
    return rne(np.cos(ang)), rne(np.sin(ang))


def rms_norm(h, w, eps) -> np.ndarray:
    """RmsNorm (src/nn/norm.rs:32-50): fp32 sum of squares, scale =
    reciprocal(sqrt(ss * (1/dim) + eps)) as two fp32 ops, RNE(RNE(h * scale) * w)."""
    h = np.asarray(h, dtype=np.float32)
    ss = np.sum(h * h, axis=-1, dtype=np.float32, keepdims=True)
    dim_inv = np.float32(1.0) / np.float32(h.shape[-1])
    root = np.sqrt(ss * dim_inv + np.float32(eps), dtype=np.float32)
    scale = (np.float32(1.0) / root).astype(np.float32)
    return rne(rne(h * scale) * np.asarray(w, dtype=np.float32))


def silu_mul(g, u) -> np.ndarray:
    """Silu (src/nn/activation.rs:19-28) times up (src/models/llama/mlp.rs:49-58):
    RNE(RNE(g / (exp(-g) + 1)) * u) in fp32."""
    g = np.asarray(g, dtype=np.float32)
    return rne(rne(g / (np.exp(-g).astype(np.float32) + np.float32(1.0))) * np.asarray(u, dtype=np.float32))


def sdpa(q, k, v, pos, scale) -> np.ndarray:
    """One head of scaled_dot_product_attention (src/nn/attention.rs:23-60)
    with the causal mask (src/nn/masking.rs:11-32): q [t, d] at positions
    pos [t], k and v [ctx, d] (ctx = max(pos) + 1). Scores RNE(q.k), times
    scale in fp32, -inf above the diagonal, fp32 softmax, probabilities RNE,
    out RNE(p . v)."""
    pos = np.asarray(pos)
    ctx = k.shape[0]
    sc = rne(np.asarray(q, np.float32) @ np.asarray(k, np.float32).T) * np.float32(scale)
    mask = np.arange(ctx)[None, :] > pos[:, None]
    sc = np.where(mask, np.float32(-np.inf), sc).astype(np.float32)
    m = sc.max(axis=-1, keepdims=True)
    e = np.exp(sc - m).astype(np.float32)
    p = rne(e / e.sum(axis=-1, dtype=np.float32, keepdims=True))
    return rne(p @ np.asarray(v, np.float32))


class RefLlama:
    """Reference-arithmetic model. `weights` supplies, per layer, dicts with
    q4 triplets 'qkv' ([q;k;v] rows), 'o', 'gate_up' ([gate;up] rows), 'down'
    and bf16 'input_norm', 'post_norm'; plus 'embed' and 'final_norm'."""

    def __init__(self, cfg, embed, layers, final_norm, max_len):
        self.cfg, self.max_len = cfg, max_len
        self.embed_q4 = embed
        self.embed_f = dequant_f32(*embed)
        self.layers = []
        for L in layers:
            self.layers.append({k: dequant_f32(*L[k]) for k in ("qkv", "o", "gate_up", "down")}
                               | {k: from_bf16(L[k]) for k in ("input_norm", "post_norm")})
        self.final_norm = from_bf16(final_norm)
        sc = cfg.rope_scaling
        scaling = None if sc is None else (sc.factor, sc.low_freq_factor, sc.high_freq_factor,
                                           sc.original_max_position_embeddings)
        self.cos, self.sin = rope_tables(cfg.head_dim, cfg.rope_theta, scaling, max_len)
        self._bf16 = {}  # id(fp32 weights) -> their materialised bf16 values, for GEMM-sized calls
        self.reset()

    def reset(self):
        c = self.cfg
        self.k = [np.zeros((c.n_kv_heads, self.max_len, c.head_dim), np.float32) for _ in self.layers]
        self.v = [np.zeros((c.n_kv_heads, self.max_len, c.head_dim), np.float32) for _ in self.layers]

    def rms_norm(self, h, w):
        return rms_norm(h, w, self.cfg.rms_norm_eps)

    def linear(self, x, w, rows=None):
        """RNE(x . w^T) in fp32, with w the fp32 dequantised weights for a
        call of at most GEMV_MAX_ROWS rows (default: x's rows) and the
        materialised bf16 weights RNE(w) above."""
        rows = x.shape[0] if rows is None else rows
        if rows > GEMV_MAX_ROWS:
            key = id(w)
            if key not in self._bf16:
                self._bf16[key] = rne(w)
            w = self._bf16[key]
        return rne(x @ w.T)

    def rope(self, x, pos):
        d = x.shape[-1] // 2
        rot = np.concatenate([-x[..., d:], x[..., :d]], axis=-1)
        c, s = self.cos[pos][:, None, :], self.sin[pos][:, None, :]
        return rne(rne(x * c) + rne(rot * s))

    def forward(self, ids, positions, batch=1, trace=None):
        """Returns the last position's logits (float32 of bf16 values). The
        sequence is one of `batch` run together: every linear call has batch
        x len(ids) rows, the LM head `batch` (one last row per sequence).
        With a dict `trace`, layer l's module outputs are stored under
        "l.<name>": qkv (the fused q/k/v projection, before RoPE), attn (the
        attention output, o_proj's input), o (o_proj's output), h_attn (the
        residual after attention), act (silu(gate) * up, down_proj's input),
        mlp (down_proj's output) and h (the layer's output); "norm" holds the
        final RMSNorm of the last row, the LM head's input."""
        c = self.cfg
        t = len(ids)
        rows = batch * t
        pos = np.asarray(positions)
        h = rne(self.embed_f[np.asarray(ids)])
        group = c.n_heads // c.n_kv_heads
        scale = np.float32(1.0) / np.sqrt(np.float32(c.head_dim), dtype=np.float32)
        for li, L in enumerate(self.layers):
            x = self.rms_norm(h, L["input_norm"])
            qkv = self.linear(x, L["qkv"], rows)
            hq, hk = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
            q = qkv[:, :hq].reshape(t, c.n_heads, c.head_dim)
            k = qkv[:, hq:hq + hk].reshape(t, c.n_kv_heads, c.head_dim)
            v = qkv[:, hq + hk:].reshape(t, c.n_kv_heads, c.head_dim)
            q, k = self.rope(q, pos), self.rope(k, pos)
            self.k[li][:, pos, :] = k.transpose(1, 0, 2)
            self.v[li][:, pos, :] = v.transpose(1, 0, 2)
            ctx = int(pos.max()) + 1
            out = np.empty((t, c.n_heads, c.head_dim), np.float32)
            for hh in range(c.n_heads):
                kv = hh // group
                out[:, hh, :] = sdpa(q[:, hh, :], self.k[li][kv, :ctx, :], self.v[li][kv, :ctx, :], pos, scale)
            a = self.linear(out.reshape(t, -1), L["o"], rows)
            h_attn = rne(h + a)
            x = self.rms_norm(h_attn, L["post_norm"])
            gu = self.linear(x, L["gate_up"], rows)
            act = silu_mul(gu[:, :c.ffn], gu[:, c.ffn:])
            mlp = self.linear(act, L["down"], rows)
            h = rne(h_attn + mlp)
            if trace is not None:
                for name, val in (("qkv", qkv), ("attn", out.reshape(t, -1)), ("o", a), ("h_attn", h_attn),
                                  ("act", act), ("mlp", mlp), ("h", h)):
                    trace[f"{li}.{name}"] = val
        x = self.rms_norm(h, self.final_norm)
        if trace is not None:
            trace["norm"] = x[-1:]
        return self.linear(x[-1:], self.embed_f, batch)[0]

    def generate(self, prompt, new_tokens, top_k=5, batch=1):
        """Greedy tokens and, per step, the top-k ids (ranked by logit, then
        by the lowest id); `batch` as in forward."""
        import time

        self.reset()
        ids = list(int(i) for i in prompt)
        t0 = time.perf_counter()
        logits = self.forward(ids, np.arange(len(ids)), batch)
        self.prefill_s = time.perf_counter() - t0
        self.first_logits = logits
        self.step_logits = [logits]  # the logits that chose each token
        tokens, tops = [], []
        t0 = time.perf_counter()
        for step in range(new_tokens):
            tokens.append(argmax(logits))
            tops.append(top_ids(logits, top_k))
            if step + 1 == new_tokens:
                break
            p = len(prompt) + step
            logits = self.forward([tokens[-1]], np.array([p]), batch)
            self.step_logits.append(logits)
        self.decode_s = time.perf_counter() - t0  # new_tokens - 1 single-token forwards
        return np.array(tokens, dtype=np.uint32), tops


def compare_close(actual, expected, atol, rtol=1e-2):
    """src/eval/compare.rs:54-91 and CloseReport::passed (:27-36): an element
    is close when |a - e| <= atol + rtol * max(|a|, |e|); non-finite elements
    on either side count against; the comparison passes when no element is
    non-finite and at least 999 per mille are close. rtol is the reference's
    RTOL (src/eval/mod.rs:53)."""
    a = np.asarray(actual, np.float32).ravel()
    e = np.asarray(expected, np.float32).ravel()
    if a.shape != e.shape:
        raise ValueError(f"element counts differ: {a.size} against {e.size}")
    finite = np.isfinite(a) & np.isfinite(e)
    err = np.abs(a - e)
    bound = np.float32(atol) + np.float32(rtol) * np.maximum(np.abs(a), np.abs(e))
    close = finite & (err <= bound)
    n, n_close, n_bad = a.size, int(np.count_nonzero(close)), int(np.count_nonzero(~finite))
    return {"numel": n, "close_count": n_close, "close_fraction": n_close / n if n else 1.0,
            "non_finite_count": n_bad, "max_abs_error": float(err[finite].max()) if finite.any() else 0.0,
            "passed": close_passed(n, n_close, n_bad)}


def close_passed(numel, close_count, non_finite_count) -> bool:
    """CloseReport::passed (src/eval/compare.rs:27-36): no non-finite element
    and close_count * 1000 >= numel * 999."""
    return non_finite_count == 0 and close_count * 1000 >= numel * 999


def module_atol(name: str) -> float:
    """src/models/llama/model.rs:362-368: by the module name's last part."""
    last = name.rsplit(".", 1)[-1]
    if last == "embed_tokens":
        return 1e-3
    if last in ("q_proj", "k_proj", "o_proj"):
        return 2e-2
    return 1e-2


def argmax(values) -> int:
    v = np.asarray(values, dtype=np.float32)
    return int(np.flatnonzero(v == v.max())[0])


def top_ids(values, k):
    v = np.asarray(values, dtype=np.float32)
    order = np.lexsort((np.arange(v.size), -v))
    return [int(i) for i in order[:k]]


def compare_generation(actual_tokens, actual_tops, expected_tokens, expected_tops):
    """src/eval/generation.rs:132-176: close when the tokens match, or when at
    the first divergence each token is in the other run's top-k."""
    n = min(len(actual_tokens), len(expected_tokens))
    first = next((i for i in range(n) if actual_tokens[i] != expected_tokens[i]), None)

    def in_top(tops, step, tok):
        return step < len(tops) and tok in tops[step]

    close = n > 0 and (first is None or (in_top(expected_tops, first, int(actual_tokens[first]))
                                         and in_top(actual_tops, first, int(expected_tokens[first]))))
    return {"compared_tokens": n, "matched_tokens": n if first is None else first,
            "first_divergence": first, "close": bool(close)}
