"""Safetensors checkpoints and their q4 weight triplets.

``Weights`` mirrors the reference's reader (src/weights/mod.rs:26-400): one
``model.safetensors`` or a ``model.safetensors.index.json`` naming shards
(plain file names only), each shard memory-mapped read-only, a tensor found
in exactly one shard, dtypes F32 / BF16 / U32 and shapes of rank <= 4 with
at most 0x7FFF_FFFF elements (src/nn/shape.rs:110-145); every other case is a
``WeightsError`` of the reference's kind. The header checks restate those of
the safetensors crate the reference pins (0.8.0, Cargo.lock:1957-1958):
an 8-byte little-endian header length of at most 100,000,000, a UTF-8 JSON
object, tensors whose byte ranges tile the data section in order with no
gap, each ``numel * dtype size`` long.

``load_tensor`` is the reference's BF16 gate (src/models/llama/weights.rs:
15-55). The q4 path adds ``load_q4_weight``: ``{name}.weight`` U32 [N, K/8]
(8 little-endian nibbles per word), ``{name}.scales`` and ``{name}.biases``
BF16 [N, K/group], each with the same not-found / dtype / shape errors.
"""
from __future__ import annotations

import json
import mmap
import os
from dataclasses import dataclass
from typing import Iterator

import numpy as np

from .primitive import DType

INDEX_FILE = "model.safetensors.index.json"
SINGLE_FILE = "model.safetensors"
HEADER_LEN_BYTES = 8
MAX_INDEX_BYTES = 100 * 1024 * 1024
MAX_HEADER_BYTES = 100_000_000
MAX_RANK = 4
MAX_NUMEL = 0x7FFF_FFFF

# safetensors dtype names and their sizes in bits (the format's table)
_DTYPE_BITS = {
    "BOOL": 8, "F4": 4, "F6_E2M3": 6, "F6_E3M2": 6, "U8": 8, "I8": 8, "F8_E5M2": 8, "F8_E4M3": 8,
    "F8_E8M0": 8, "I16": 16, "U16": 16, "F16": 16, "BF16": 16, "I32": 32, "U32": 32, "F32": 32,
    "C64": 64, "F64": 64, "I64": 64, "U64": 64,
}
# the dtypes Foundry reads (src/weights/mod.rs:357-365)
_FOUNDRY_DTYPES = {"F32": DType.F32, "BF16": DType.BF16, "U32": DType.U32}
_NUMPY = {DType.F32: np.float32, DType.BF16: np.uint16, DType.U32: np.uint32}


class WeightsError(Exception):
    """src/weights/error.rs: kind is the reference's variant name."""

    def __init__(self, kind: str, message: str = ""):
        super().__init__(f"{kind}: {message}" if message else kind)
        self.kind = kind


class LlamaError(Exception):
    """LlamaError / LlamaConfigError (src/models/llama/error.rs)."""

    def __init__(self, kind: str, message: str = ""):
        super().__init__(f"{kind}: {message}" if message else kind)
        self.kind = kind


@dataclass(frozen=True)
class Shard:
    name: str
    bytes: object  # bytes, bytearray, mmap or memoryview


@dataclass(frozen=True)
class WeightView:
    name: str
    dtype: DType
    shape: tuple
    bytes: memoryview

    def __eq__(self, other):
        return (isinstance(other, WeightView) and (self.name, self.dtype, self.shape) ==
                (other.name, other.dtype, other.shape) and bytes(self.bytes) == bytes(other.bytes))

    def numpy(self) -> np.ndarray:
        return np.frombuffer(self.bytes, dtype=_NUMPY[self.dtype]).reshape(self.shape)


@dataclass(frozen=True)
class _Entry:
    dtype: DType
    shape: tuple
    shard: int
    start: int
    stop: int


def check_shard_name(name: str) -> None:
    """A shard is named by a plain file name (src/weights/mod.rs:251-258)."""
    if not name or name in (".", "..") or os.path.basename(name) != name or "/" in name or "\\" in name:
        raise WeightsError("InvalidShardName", repr(name))


def _shape(dims) -> tuple:
    """Shape::try_from (src/nn/shape.rs:110-145): rank <= 4, numel <= 2^31 - 1."""
    dims = tuple(int(d) for d in dims)
    if len(dims) > MAX_RANK:
        raise WeightsError("InvalidShape", f"rank {len(dims)}")
    numel = 1
    for d in dims:
        if d != 0:
            numel *= d
            if numel > MAX_NUMEL:
                raise WeightsError("InvalidShape", f"{dims} has too many elements")
    return dims


def read_metadata(buf) -> tuple[int, list]:
    """The safetensors header of one file: (header length, [(name, dtype
    name, shape, (begin, end))]) with offsets relative to the data section;
    any violation is InvalidHeader."""
    view = memoryview(buf)
    if len(view) < HEADER_LEN_BYTES:
        raise WeightsError("InvalidHeader", "file shorter than the header length")
    n = int.from_bytes(view[:HEADER_LEN_BYTES], "little")
    if n > MAX_HEADER_BYTES:
        raise WeightsError("InvalidHeader", f"header of {n} bytes")
    if HEADER_LEN_BYTES + n > len(view):
        raise WeightsError("InvalidHeader", "header past the end of the file")
    try:
        text = bytes(view[HEADER_LEN_BYTES:HEADER_LEN_BYTES + n]).decode("utf-8")
        header = json.loads(text)
    except (UnicodeDecodeError, ValueError) as e:
        raise WeightsError("InvalidHeader", str(e)) from None
    if not isinstance(header, dict):
        raise WeightsError("InvalidHeader", "header is not a JSON object")
    tensors = []
    for name, info in header.items():
        if name == "__metadata__":
            if not isinstance(info, dict) or not all(isinstance(v, str) for v in info.values()):
                raise WeightsError("InvalidHeader", "__metadata__ is not a map of strings")
            continue
        if not isinstance(info, dict) or not {"dtype", "shape", "data_offsets"} <= set(info):
            raise WeightsError("InvalidHeader", f"tensor {name!r} entry")
        dtype, shape, offsets = info["dtype"], info["shape"], info["data_offsets"]
        if dtype not in _DTYPE_BITS:
            raise WeightsError("InvalidHeader", f"dtype {dtype!r}")
        if (not isinstance(shape, list) or not all(isinstance(d, int) and not isinstance(d, bool) and d >= 0
                                                     for d in shape)):
            raise WeightsError("InvalidHeader", f"tensor {name!r} shape")
        if (not isinstance(offsets, list) or len(offsets) != 2 or
                not all(isinstance(o, int) and not isinstance(o, bool) and o >= 0 for o in offsets)):
            raise WeightsError("InvalidHeader", f"tensor {name!r} offsets")
        tensors.append((name, dtype, shape, (offsets[0], offsets[1])))
    # the byte ranges tile the data section in order, each exactly numel * size
    end = 0
    for name, dtype, shape, (b, e) in sorted(tensors, key=lambda t: t[3]):
        if b != end or e < b:
            raise WeightsError("InvalidHeader", f"tensor {name!r} offsets do not follow the previous tensor")
        numel = 1
        for d in shape:
            numel *= d
        bits = numel * _DTYPE_BITS[dtype]
        if bits % 8 != 0 or bits // 8 != e - b:
            raise WeightsError("InvalidHeader", f"tensor {name!r} has {e - b} bytes for {shape} {dtype}")
        end = e
    if HEADER_LEN_BYTES + n + end != len(view):
        raise WeightsError("InvalidHeader", "the data section is not covered exactly")
    return n, tensors


class Weights:
    """Tensors of one safetensors checkpoint, by name (src/weights/mod.rs:42-212)."""

    def __init__(self, shards: list, tensors: dict, total_size):
        self._shards = shards
        self._tensors = tensors
        self._total_size = total_size

    @classmethod
    def open(cls, directory) -> "Weights":
        index_path = os.path.join(directory, INDEX_FILE)
        index = None
        if os.path.isfile(index_path):
            try:
                size = os.path.getsize(index_path)
                if size > MAX_INDEX_BYTES:
                    raise WeightsError("IndexTooLarge", f"{size} bytes")
                with open(index_path, "rb") as f:
                    index = _parse_index(f.read())
            except OSError as e:
                raise WeightsError("IndexRead", str(e)) from None
        names = sorted(set(index["weight_map"].values())) if index else [SINGLE_FILE]
        shards = []
        for name in names:
            check_shard_name(name)
            path = os.path.join(directory, name)
            try:
                with open(path, "rb") as f:
                    data = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if os.path.getsize(path) else b""
            except OSError as e:
                raise WeightsError("ShardOpen", f"{path}: {e}") from None
            shards.append(Shard(name, data))
        return cls._assemble(index, shards)

    @classmethod
    def from_shards(cls, index: bytes | None, shards: list) -> "Weights":
        return cls._assemble(None if index is None else _parse_index(index), shards)

    @classmethod
    def _assemble(cls, index, shards: list) -> "Weights":
        tensors = {}
        for si, shard in enumerate(shards):
            n, entries = read_metadata(shard.bytes)
            data_start = HEADER_LEN_BYTES + n
            for name, dtype, shape, (b, e) in entries:
                if dtype not in _FOUNDRY_DTYPES:
                    raise WeightsError("UnknownDType", f"tensor {name!r} is {dtype}")
                entry = _Entry(_FOUNDRY_DTYPES[dtype], _shape(shape), si, data_start + b, data_start + e)
                if name in tensors:
                    raise WeightsError("DuplicateTensor", name)
                tensors[name] = entry
        if index is not None:
            for name, shard in index["weight_map"].items():
                entry = tensors.get(name)
                if entry is None or shards[entry.shard].name != shard:
                    raise WeightsError("IndexMismatch", f"{name} -> {shard}")
        total = index.get("metadata", {}) if index else None
        total_size = total.get("total_size") if isinstance(total, dict) else None
        return cls(shards, tensors, total_size)

    def tensor(self, name: str) -> WeightView | None:
        entry = self._tensors.get(name)
        if entry is None:
            return None
        data = memoryview(self._shards[entry.shard].bytes)[entry.start:entry.stop]
        return WeightView(name, entry.dtype, entry.shape, data)

    def tensors(self) -> Iterator[WeightView]:
        for name in self._tensors:
            yield self.tensor(name)

    @property
    def shard_count(self) -> int:
        return len(self._shards)

    @property
    def total_size(self):
        return self._total_size

    def nbytes(self) -> int:
        n = sum(e.stop - e.start for e in self._tensors.values())
        if n >= 1 << 64:
            raise WeightsError("ByteCountOverflow")
        if self._total_size is not None and n != self._total_size:
            raise WeightsError("ByteCountMismatch", f"{n} bytes, index declares {self._total_size}")
        return n

    def numel(self) -> int:
        total = 0
        for e in self._tensors.values():
            n = 0 if 0 in e.shape else int(np.prod(e.shape, dtype=np.uint64)) if e.shape else 1
            total += n
        if total >= 1 << 64:
            raise WeightsError("ParameterCountOverflow")
        return total


def _parse_index(data: bytes) -> dict:
    """model.safetensors.index.json: {"metadata": {"total_size"}?, "weight_map": {tensor: shard}}."""
    try:
        index = json.loads(bytes(data).decode("utf-8"))
    except (UnicodeDecodeError, ValueError) as e:
        raise WeightsError("IndexJson", str(e)) from None
    wm = index.get("weight_map") if isinstance(index, dict) else None
    if not isinstance(wm, dict) or not all(isinstance(k, str) and isinstance(v, str) for k, v in wm.items()):
        raise WeightsError("IndexJson", "weight_map is not a map of strings")
    md = index.get("metadata")
    if md is not None and (not isinstance(md, dict) or
                           (md.get("total_size") is not None and not isinstance(md.get("total_size"), int))):
        raise WeightsError("IndexJson", "metadata")
    return index


# ---- model-facing loads (src/models/llama/weights.rs:15-55) ----

def checked_view(view: WeightView | None, name: str, dims_expected, dtype: DType = DType.BF16) -> WeightView:
    if view is None:
        raise LlamaError("TensorNotFound", name)
    if view.dtype != dtype:
        raise LlamaError("TensorDTypeMismatch", f"{name} is {view.dtype.name}, expected {dtype.name}")
    if tuple(view.shape) != tuple(dims_expected):
        raise LlamaError("TensorShapeMismatch", f"{name} is {view.shape}, expected {tuple(dims_expected)}")
    return view


def load_tensor(device, weights: Weights, name: str, dims_expected):
    """A BF16 tensor of the expected shape on the device (load_tensor)."""
    from .tensor import Tensor
    view = checked_view(weights.tensor(name), name, dims_expected)
    return Tensor.from_bytes(device, bytes(view.bytes), view.dtype, view.shape)


def q4_views(weights: Weights, name: str, n: int, k: int, group: int = 64):
    """The checked q4 triplet of weight `name` ([n, k] logical): views of
    {name}.weight U32 [n, k/8], {name}.scales and {name}.biases BF16
    [n, k/group]."""
    if k % 8 != 0 or k % group != 0:
        raise LlamaError("TensorShapeMismatch", f"{name}: k={k} is not a multiple of 8 and {group}")
    wq = checked_view(weights.tensor(f"{name}.weight"), f"{name}.weight", (n, k // 8), DType.U32)
    s = checked_view(weights.tensor(f"{name}.scales"), f"{name}.scales", (n, k // group))
    b = checked_view(weights.tensor(f"{name}.biases"), f"{name}.biases", (n, k // group))
    return wq, s, b


def load_q4_weight(device, weights: Weights, name: str, n: int, k: int, group: int = 64):
    """The q4 triplet of weight `name` on the device, as a Q4Weight."""
    from .nn import Q4Weight
    from .tensor import Tensor
    views = q4_views(weights, name, n, k, group)
    wq, s, b = (Tensor.from_bytes(device, bytes(v.bytes), v.dtype, v.shape) for v in views)
    return Q4Weight(wq, s, b, group)


# ---- Llama checkpoints (names of src/models/llama/{model,attention,mlp}.rs) ----

def llama_embed_name() -> str:
    return "model.embed_tokens"


def llama_layer_names(layer: int) -> dict:
    p = f"model.layers.{layer}"
    return {"q": f"{p}.self_attn.q_proj", "k": f"{p}.self_attn.k_proj", "v": f"{p}.self_attn.v_proj",
            "o": f"{p}.self_attn.o_proj", "gate": f"{p}.mlp.gate_proj", "up": f"{p}.mlp.up_proj",
            "down": f"{p}.mlp.down_proj", "input_norm": f"{p}.input_layernorm.weight",
            "post_norm": f"{p}.post_attention_layernorm.weight"}


def _triplet(weights: Weights, name: str, n: int, k: int):
    return tuple(v.numpy() for v in q4_views(weights, name, n, k))


def llama_q4_layer(weights: Weights, cfg, layer: int) -> dict:
    """One layer's host arrays in the layout the decoder uses: [q; k; v] and
    [gate; up] rows concatenated (each output row depends only on its own
    weight row), plus the two norm weights."""
    nm = llama_layer_names(layer)
    hq, hkv, h, f = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.hidden, cfg.ffn
    q, k, v = (_triplet(weights, nm[x], rows, h) for x, rows in (("q", hq), ("k", hkv), ("v", hkv)))
    gate, up = (_triplet(weights, nm[x], f, h) for x in ("gate", "up"))
    out = {
        "qkv": tuple(np.concatenate([a, b2, c]) for a, b2, c in zip(q, k, v)),
        "o": _triplet(weights, nm["o"], h, hq),
        "gate_up": tuple(np.concatenate([a, b2]) for a, b2 in zip(gate, up)),
        "down": _triplet(weights, nm["down"], h, f),
    }
    for key in ("input_norm", "post_norm"):
        out[key] = checked_view(weights.tensor(nm[key]), nm[key], (h,)).numpy()
    return out


def llama_q4_embed(weights: Weights, cfg):
    return _triplet(weights, llama_embed_name(), cfg.vocab, cfg.hidden)


def llama_final_norm(weights: Weights, cfg) -> np.ndarray:
    return checked_view(weights.tensor("model.norm.weight"), "model.norm.weight", (cfg.hidden,)).numpy()


def serialize(tensors: dict, metadata: dict | None = None) -> bytes:
    """A safetensors file of {name: (dtype name, shape, raw bytes)}, tensors
    in name order."""
    header, data, off = {}, [], 0
    if metadata:
        header["__metadata__"] = dict(metadata)
    for name in sorted(tensors):
        dtype, shape, raw = tensors[name]
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        data.append(bytes(raw))
        off += len(raw)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    return len(h).to_bytes(8, "little") + h + b"".join(data)


def save_q4_llama(directory, cfg, embed, layers, final_norm, shards: int = 1) -> None:
    """Writes a q4 Llama checkpoint: config.json and model.safetensors (or an
    index and `shards` shard files). embed: (wq, s, b); layers: per layer the
    decoder's dict (qkv, o, gate_up, down triplets; input_norm, post_norm)."""
    os.makedirs(directory, exist_ok=True)
    hq, hkv, f = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.ffn
    tensors = {}

    def put_q4(name, trip):
        wq, s, b = trip
        tensors[f"{name}.weight"] = ("U32", wq.shape, np.ascontiguousarray(wq, np.uint32).tobytes())
        tensors[f"{name}.scales"] = ("BF16", s.shape, np.ascontiguousarray(s, np.uint16).tobytes())
        tensors[f"{name}.biases"] = ("BF16", b.shape, np.ascontiguousarray(b, np.uint16).tobytes())

    put_q4(llama_embed_name(), embed)
    for li, L in enumerate(layers):
        nm = llama_layer_names(li)
        rows = {"q": (0, hq), "k": (hq, hq + hkv), "v": (hq + hkv, hq + 2 * hkv)}
        for x, (a, b2) in rows.items():
            put_q4(nm[x], tuple(t[a:b2] for t in L["qkv"]))
        put_q4(nm["o"], L["o"])
        put_q4(nm["gate"], tuple(t[:f] for t in L["gate_up"]))
        put_q4(nm["up"], tuple(t[f:] for t in L["gate_up"]))
        put_q4(nm["down"], L["down"])
        for key in ("input_norm", "post_norm"):
            tensors[nm[key]] = ("BF16", L[key].shape, np.ascontiguousarray(L[key], np.uint16).tobytes())
    tensors["model.norm.weight"] = ("BF16", final_norm.shape, np.ascontiguousarray(final_norm, np.uint16).tobytes())
    names = sorted(tensors)
    if shards <= 1:
        with open(os.path.join(directory, SINGLE_FILE), "wb") as fh:
            fh.write(serialize(tensors, {"format": "q4-affine-g64"}))
    else:
        weight_map, total = {}, 0
        for si in range(shards):
            part = {n: tensors[n] for n in names[si::shards]}
            sname = f"model-{si + 1:05d}-of-{shards:05d}.safetensors"
            with open(os.path.join(directory, sname), "wb") as fh:
                fh.write(serialize(part))
            for n in part:
                weight_map[n] = sname
                total += len(part[n][2])
        with open(os.path.join(directory, INDEX_FILE), "w") as fh:
            json.dump({"metadata": {"total_size": total}, "weight_map": weight_map}, fh)
    rs = cfg.rope_scaling
    config = {
        "model_type": "llama", "hidden_size": cfg.hidden, "intermediate_size": cfg.ffn,
        "num_hidden_layers": cfg.n_layers, "num_attention_heads": cfg.n_heads,
        "num_key_value_heads": cfg.n_kv_heads, "head_dim": cfg.head_dim, "rms_norm_eps": cfg.rms_norm_eps,
        "rope_theta": cfg.rope_theta, "max_position_embeddings": cfg.max_position_embeddings,
        "vocab_size": cfg.vocab, "tie_word_embeddings": True, "eos_token_id": list(cfg.eos_token_id) or [0],
        "rope_scaling": None if rs is None else {
            "rope_type": "llama3", "factor": rs.factor, "low_freq_factor": rs.low_freq_factor,
            "high_freq_factor": rs.high_freq_factor,
            "original_max_position_embeddings": rs.original_max_position_embeddings},
        "quantization": {"group_size": 64, "bits": 4},
    }
    with open(os.path.join(directory, "config.json"), "w") as fh:
        json.dump(config, fh, indent=1)
