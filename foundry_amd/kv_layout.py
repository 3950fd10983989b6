"""Host-side view of the K cache layout the attention entry points use.

`fh_rope_kv`, `fh_attention`, `fh_decode_attention` (and the decoder built on
them) keep each (sequence, KV head)'s keys in groups of 16: group g holds keys
16 g .. 16 g + n_g - 1 (n_g = min(16, max_len - 16 g)) as n_g * head_dim
contiguous elements laid out [head_dim / 32][n_g][32]. A matrix-core fragment
of 16 keys x 32 dims is then one 1 KB run. The region of one (sequence, KV
head) is still max_len * head_dim elements, so cache sizes do not change; only
the order inside the region does. V caches keep [max_len, head_dim].

These helpers convert numpy arrays of keys [..., max_len, head_dim] (the
StaticCache layout, src/nn/kv_cache.rs:41-80) to and from that order, for
callers that fill or read a cache from the host.
"""
import numpy as np


def k_tile_index(max_len: int, head_dim: int) -> np.ndarray:
    """[max_len, head_dim] array: the element offset, inside one (sequence,
    KV head) region, of key j's dim d."""
    if head_dim % 32 != 0:
        raise ValueError("head_dim must be a multiple of 32")
    j = np.arange(max_len, dtype=np.int64)[:, None]
    d = np.arange(head_dim, dtype=np.int64)[None, :]
    g = j // 16
    n_g = np.minimum(16, max_len - 16 * g)
    return g * 16 * head_dim + (d // 32) * n_g * 32 + (j % 16) * 32 + d % 32


def tile_k(k: np.ndarray) -> np.ndarray:
    """Keys [..., max_len, head_dim] -> an array of the same shape whose
    memory (C order) is the tiled layout of each [max_len, head_dim] region."""
    *lead, max_len, head_dim = k.shape
    idx = k_tile_index(max_len, head_dim).ravel()
    flat = np.ascontiguousarray(k).reshape(*lead, max_len * head_dim)
    out = np.empty_like(flat)
    out[..., idx] = flat
    return out.reshape(k.shape)


def untile_k(t: np.ndarray) -> np.ndarray:
    """Inverse of tile_k: a tiled cache read back from the device, in
    [..., max_len, head_dim] order."""
    *lead, max_len, head_dim = t.shape
    idx = k_tile_index(max_len, head_dim).ravel()
    flat = np.ascontiguousarray(t).reshape(*lead, max_len * head_dim)
    return flat[..., idx].reshape(t.shape)
