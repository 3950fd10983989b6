"""Checkpoint reading (foundry_amd/weights.py) and config parsing, on the CPU.

The cases restate the reference's own tests of the reader
(src/weights/mod.rs:410-900) and of LlamaConfig (src/models/llama/
config.rs:284-460) with the same inputs and expected errors. Files are built
by hand where the reference builds them by hand, and otherwise by the
`safetensors` package. That package (0.8.0) wraps the Rust crate version the
reference pins (Cargo.lock:1957-1958), so its deserialize is the reference's
own header parser: every header ours rejects as InvalidHeader it rejects too,
every file ours reads it reads, and it reads back what our writer writes.
"""
import json
import struct
from dataclasses import replace

import numpy as np
import pytest
import safetensors
from safetensors import deserialize as st_deserialize
from safetensors.numpy import save as st_save

from foundry_amd import synth
from foundry_amd.llama import LlamaConfig, embed_weights, final_norm_weight, layer_weights
from foundry_amd.primitive import DType
from foundry_amd.weights import (LlamaError, Shard, WeightView, Weights, WeightsError, check_shard_name,
                                 checked_view, llama_final_norm, llama_q4_embed, llama_q4_layer, q4_views,
                                 save_q4_llama, serialize)

TINY = LlamaConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000)


def one(data, name="model.safetensors"):
    return Weights.from_shards(None, [Shard(name, data)])


def file_of(header: bytes, data: bytes = b"") -> bytes:
    return struct.pack("<Q", len(header)) + header + data


def test_valid_file_returns_dtype_shape_and_bytes():
    header = json.dumps({"__metadata__": {"format": "pt"},
                         "a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 12]},
                         "b": {"dtype": "F32", "shape": [4], "data_offsets": [12, 28]}}).encode()
    w = one(file_of(header, bytes(range(28))))
    assert w.tensor("a") == WeightView("a", DType.BF16, (2, 3), memoryview(bytes(range(12))))
    assert w.tensor("b") == WeightView("b", DType.F32, (4,), memoryview(bytes(range(12, 28))))
    assert len(list(w.tensors())) == 2  # metadata is not a tensor
    assert w.shard_count == 1 and w.total_size is None


def _shard(name, arrays):
    return Shard(name, st_save(arrays))


def test_index_with_two_shards_loads_both():
    s1 = _shard("s1.safetensors", {"a": np.array([1, 2], np.float32)})
    s2 = _shard("s2.safetensors", {"b": np.array([3], np.uint32)})
    index = json.dumps({"metadata": {"total_size": 12},
                        "weight_map": {"a": "s1.safetensors", "b": "s2.safetensors"}}).encode()
    w = Weights.from_shards(index, [s1, s2])
    assert w.shard_count == 2 and w.total_size == 12 and w.nbytes() == 12 and w.numel() == 3
    assert w.tensor("a").numpy().tolist() == [1.0, 2.0] and w.tensor("b").numpy().tolist() == [3]


@pytest.mark.parametrize("shard", ["s2.safetensors", "missing.safetensors"])
def test_index_naming_the_wrong_shard_is_rejected(shard):
    s1 = _shard("s1.safetensors", {"a": np.zeros(1, np.float32)})
    s2 = _shard("s2.safetensors", {"b": np.zeros(1, np.float32)})
    index = json.dumps({"weight_map": {"a": shard}}).encode()
    with pytest.raises(WeightsError) as e:
        Weights.from_shards(index, [s1, s2])
    assert e.value.kind == "IndexMismatch"


def test_index_without_metadata_declares_no_size():
    s1 = _shard("s1.safetensors", {"a": np.zeros(2, np.float32)})
    w = Weights.from_shards(json.dumps({"weight_map": {"a": "s1.safetensors"}}).encode(), [s1])
    assert w.total_size is None and w.nbytes() == 8


def test_declared_size_mismatch_is_rejected():
    s1 = _shard("s1.safetensors", {"a": np.zeros(2, np.float32)})
    w = Weights.from_shards(json.dumps({"metadata": {"total_size": 9}, "weight_map": {"a": "s1.safetensors"}})
                            .encode(), [s1])
    with pytest.raises(WeightsError) as e:
        w.nbytes()
    assert e.value.kind == "ByteCountMismatch"


def test_invalid_index_json_is_rejected():
    with pytest.raises(WeightsError) as e:
        Weights.from_shards(b"{", [])
    assert e.value.kind == "IndexJson"


def test_duplicate_tensor_across_shards_is_rejected():
    shards = [_shard(f"s{i}.safetensors", {"a": np.zeros(1, np.float32)}) for i in (1, 2)]
    with pytest.raises(WeightsError) as e:
        Weights.from_shards(None, shards)
    assert e.value.kind == "DuplicateTensor"


def test_shard_names_with_a_path_are_rejected():
    for name in ["a/b", "", "..", "../s1.safetensors"]:
        with pytest.raises(WeightsError) as e:
            check_shard_name(name)
        assert e.value.kind == "InvalidShardName", name
    check_shard_name("s1.safetensors")


@pytest.mark.parametrize("header", [b"{", b"[]", b"null", b"\xff"])
def test_header_rejected_by_the_parser_is_invalid(header):
    with pytest.raises(WeightsError) as e:
        one(file_of(header))
    assert e.value.kind == "InvalidHeader"


def test_pinned_crate_is_the_reference_version():
    assert safetensors.__version__ == "0.8.0"


def test_header_checks_of_the_format():
    """Offsets that leave a gap, overlap, or disagree with dtype x shape, and
    a data section longer than the tensors, are invalid headers."""
    cases = [{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}},
             {"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}},
             {"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},
              "b": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}},
             {"a": {"dtype": "Q4", "shape": [1], "data_offsets": [0, 4]}}]
    files = [file_of(json.dumps(h).encode(), bytes(8)) for h in cases]
    # 8 data bytes for a 4-byte tensor
    files.append(file_of(json.dumps({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}).encode(), bytes(8)))
    files += [file_of(h) for h in (b"{", b"[]", b"null", b"\xff")]
    for f in files:
        with pytest.raises(WeightsError) as e:
            one(f)
        assert e.value.kind == "InvalidHeader", f[:80]
        with pytest.raises(Exception):
            st_deserialize(f)  # the pinned crate rejects it as well


@pytest.mark.parametrize("arr", [np.zeros(1, np.int64), np.zeros(4, np.float16)])
def test_unknown_dtype_is_rejected(arr):
    with pytest.raises(WeightsError) as e:
        one(st_save({"a": arr}))
    assert e.value.kind == "UnknownDType"


def test_u32_dtype_is_accepted():
    assert one(st_save({"b": np.zeros(1, np.uint32)})).tensor("b").dtype == DType.U32


def test_invalid_tensor_shape_is_rejected():
    with pytest.raises(WeightsError) as e:
        one(st_save({"a": np.zeros((1, 1, 1, 1, 1), np.float32)}))
    assert e.value.kind == "InvalidShape"


def test_empty_header_has_no_tensors():
    assert list(one(file_of(b"{}")).tensors()) == []


def test_scalar_and_zero_dim_tensors_are_accepted():
    w = one(st_save({"s": np.array(1.5, np.float32), "z": np.zeros((0, 3), np.float32)}))
    assert w.tensor("s").shape == () and w.tensor("z").shape == (0, 3) and w.numel() == 1


def test_our_writer_reads_back_with_the_safetensors_package():
    wq = synth.q4_weights(5, 32, 128)[0]
    raw = serialize({"w": ("U32", wq.shape, wq.tobytes()), "n": ("BF16", (3,), np.arange(3, dtype=np.uint16).tobytes())},
                    {"format": "q4"})
    back = {name: info for name, info in st_deserialize(raw)}
    assert back["w"]["dtype"] == "U32" and back["w"]["shape"] == list(wq.shape)
    assert bytes(back["w"]["data"]) == wq.tobytes()
    assert back["n"]["dtype"] == "BF16" and bytes(back["n"]["data"]) == np.arange(3, dtype=np.uint16).tobytes()
    assert np.array_equal(one(raw).tensor("w").numpy(), wq)


# ---------------- config (src/models/llama/config.rs:230-460) ----------------

def instruct_config() -> dict:
    return {"architectures": ["LlamaForCausalLM"], "attention_bias": False, "attention_dropout": 0.0,
            "bos_token_id": 128000, "eos_token_id": [128001, 128008, 128009], "head_dim": 128, "hidden_act": "silu",
            "hidden_size": 3072, "initializer_range": 0.02, "intermediate_size": 8192,
            "max_position_embeddings": 131072, "mlp_bias": False, "model_type": "llama", "num_attention_heads": 24,
            "num_hidden_layers": 28, "num_key_value_heads": 8, "pretraining_tp": 1, "rms_norm_eps": 1e-05,
            "rope_scaling": {"factor": 32.0, "high_freq_factor": 4.0, "low_freq_factor": 1.0,
                             "original_max_position_embeddings": 8192, "rope_type": "llama3"},
            "rope_theta": 500000.0, "tie_word_embeddings": True, "torch_dtype": "bfloat16",
            "transformers_version": "4.45.0.dev0", "use_cache": True, "vocab_size": 128256}


def parse(cfg):
    return LlamaConfig.parse(json.dumps(cfg).encode())


def with_(cfg, key, value):
    c = dict(cfg)
    if value is KeyError:
        c.pop(key)
    else:
        c[key] = value
    return c


def test_instruct_values_are_accepted():
    c = parse(instruct_config())
    assert (c.hidden, c.ffn, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim) == (3072, 8192, 28, 24, 8, 128)
    assert c.rms_norm_eps == np.float32(1e-5) and c.rope_theta == 500000.0
    assert c.rope_scaling.factor == 32.0 and c.rope_scaling.low_freq_factor == 1.0
    assert c.rope_scaling.high_freq_factor == 4.0 and c.rope_scaling.original_max_position_embeddings == 8192
    assert c.max_position_embeddings == 131072 and c.vocab == 128256 and c.eos_token_id == (128001, 128008, 128009)
    assert c == replace(LlamaConfig.llama_3_2_3b(), eos_token_id=(128001, 128008, 128009),
                        rms_norm_eps=float(np.float32(1e-5)))  # the reference keeps eps as f32


def test_single_eos_token_id_becomes_a_list():
    assert parse(with_(instruct_config(), "eos_token_id", 128001)).eos_token_id == (128001,)


@pytest.mark.parametrize("key,value,kind", [
    ("model_type", "qwen3", "ModelType"),
    ("hidden_size", 3000, "HiddenSizeMismatch"),
    ("num_key_value_heads", 5, "HeadRatio"),
    ("num_key_value_heads", 0, "HeadRatio"),
    ("tie_word_embeddings", False, "UntiedEmbeddings"),
    ("hidden_size", "3072", "ConfigJson"),
    ("vocab_size", KeyError, "ConfigJson"),
])
def test_config_errors(key, value, kind):
    with pytest.raises(LlamaError) as e:
        parse(with_(instruct_config(), key, value))
    assert e.value.kind == kind


def test_other_rope_type_is_rejected():
    cfg = instruct_config()
    cfg["rope_scaling"] = dict(cfg["rope_scaling"], rope_type="linear")
    with pytest.raises(LlamaError) as e:
        parse(cfg)
    assert e.value.kind == "RopeType"


def test_null_rope_scaling_and_missing_head_dim():
    c = parse(with_(with_(instruct_config(), "rope_scaling", None), "head_dim", KeyError))
    assert c.rope_scaling is None and c.head_dim == 128
    with pytest.raises(LlamaError) as e:
        parse(with_(with_(instruct_config(), "head_dim", KeyError), "hidden_size", 3073))
    assert e.value.kind == "HiddenSizeMismatch"


# ---------------- q4 checkpoints ----------------

def test_checked_view_errors():
    w = one(serialize({"n": ("BF16", (4,), bytes(8)), "f": ("F32", (4,), bytes(16))}))
    with pytest.raises(LlamaError) as e:
        checked_view(w.tensor("missing"), "missing", (4,))
    assert e.value.kind == "TensorNotFound"
    with pytest.raises(LlamaError) as e:
        checked_view(w.tensor("f"), "f", (4,))
    assert e.value.kind == "TensorDTypeMismatch"
    with pytest.raises(LlamaError) as e:
        checked_view(w.tensor("n"), "n", (2, 2))
    assert e.value.kind == "TensorShapeMismatch"
    assert checked_view(w.tensor("n"), "n", (4,)).dtype == DType.BF16


def _bf16_file(tensors):
    return serialize({k: ("BF16" if v.dtype == np.uint16 else "U32", v.shape, v.tobytes()) for k, v in tensors.items()})


def test_q4_triplet_checks():
    wq, s, b = synth.q4_weights(3, 16, 128)
    w = one(_bf16_file({"p.weight": wq, "p.scales": s, "p.biases": b}))
    got = q4_views(w, "p", 16, 128)
    assert all(np.array_equal(g.numpy(), x) for g, x in zip(got, (wq, s, b)))
    with pytest.raises(LlamaError) as e:
        q4_views(w, "p", 16, 256)
    assert e.value.kind == "TensorShapeMismatch"
    w2 = one(_bf16_file({"p.weight": wq, "p.scales": s}))
    with pytest.raises(LlamaError) as e:
        q4_views(w2, "p", 16, 128)
    assert e.value.kind == "TensorNotFound"
    w3 = one(_bf16_file({"p.weight": wq.view(np.uint16)[:, :16].copy(), "p.scales": s, "p.biases": b}))
    with pytest.raises(LlamaError) as e:
        q4_views(w3, "p", 16, 128)
    assert e.value.kind == "TensorDTypeMismatch"


@pytest.mark.parametrize("shards", [1, 3])
def test_q4_llama_checkpoint_round_trip(tmp_path, shards):
    """save_q4_llama then Weights.open / LlamaConfig.open give back the
    decoder's arrays bit for bit (q/k/v and gate/up split and re-joined)."""
    seed = 4
    layers = [layer_weights(TINY, seed, l) for l in range(TINY.n_layers)]
    embed, norm = embed_weights(TINY, seed), final_norm_weight(TINY, seed)
    save_q4_llama(tmp_path, TINY, embed, layers, norm, shards=shards)
    cfg = LlamaConfig.open(tmp_path)
    assert (cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab) == \
        (TINY.n_layers, TINY.hidden, TINY.n_heads, TINY.n_kv_heads, TINY.head_dim, TINY.ffn, TINY.vocab)
    assert cfg.rope_scaling == TINY.rope_scaling and cfg.rope_theta == TINY.rope_theta
    w = Weights.open(tmp_path)
    assert w.shard_count == shards and (shards == 1 or w.nbytes() == w.total_size)
    for got, want in zip(llama_q4_embed(w, cfg), embed):
        assert np.array_equal(got, want)
    assert np.array_equal(llama_final_norm(w, cfg), norm)
    for l in range(TINY.n_layers):
        g = llama_q4_layer(w, cfg, l)
        for key in ("qkv", "o", "gate_up", "down"):
            assert all(np.array_equal(a, b) for a, b in zip(g[key], layers[l][key])), (l, key)
        for key in ("input_norm", "post_norm"):
            assert np.array_equal(g[key], layers[l][key])
