"""The model-directory runtime on the host: HF::Gemma::load over a Hugging
Face Gemma directory (Generation/Gemma.cpp:64-84) and ModelFiles::fromDirectory
(Model/ModelFiles.cpp:77-99), restating the reference's refusals and its
generation_config rule (GemmaConfig.cpp:204-223).  Nothing here touches a
GPU: load maps the shards and reads the tokenizer, prepare is where the
device comes in.
"""
import json
import shutil

import numpy as np
import pytest

from huggingfaceeacp_amd import gemma_q8 as G
from test_gpu_checkpoint import checkpoint_dims, checkpoint_name, write_shard

GOLDEN_TOKENIZER = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                              "MiniTokenizer.json")


def tiny_shape():
    # width 128, 2 heads of 64 over one KV head, FFN 256, vocabulary 1000
    return G.DecoderShape(128, 2, 1, 64, 2, 256, 1000, 64, 16)


def config_for(shape, **overrides):
    config = {"model_type": "gemma", "vocab_size": shape.vocab, "hidden_size": shape.width,
              "intermediate_size": shape.intermediate, "num_hidden_layers": shape.layers,
              "num_attention_heads": shape.heads, "num_key_value_heads": shape.kv_heads,
              "head_dim": shape.head_dim, "max_position_embeddings": shape.max_positions,
              "rms_norm_eps": 1e-6, "rope_theta": 10000.0, "bos_token_id": 2, "eos_token_id": 1,
              "pad_token_id": 0, "tie_word_embeddings": True}
    config.update(overrides)
    return config


def zero_tensors(shape):
    return {checkpoint_name(shape, i): ("F32", checkpoint_dims(shape, i),
                                        np.zeros(shape.tensor_elements(i), np.float32).tobytes())
            for i in range(shape.tensor_count())}


def model_directory(root, shape, sharded=False, generation=None, tokenizer=True, config=None):
    root.mkdir(parents=True, exist_ok=True)
    (root / "config.json").write_text(json.dumps(config or config_for(shape)))
    if generation is not None:
        (root / "generation_config.json").write_text(json.dumps(generation))
    if tokenizer:
        shutil.copy(GOLDEN_TOKENIZER, root / "tokenizer.json")
    tensors = zero_tensors(shape)
    if sharded:
        names = sorted(tensors)
        halves = [dict((n, tensors[n]) for n in names[1::2]), dict((n, tensors[n]) for n in names[::2])]
        files = ["model-00002-of-00002.safetensors", "model-00001-of-00002.safetensors"]
        weight_map = {}
        for file, part in zip(files, halves):
            write_shard(root / file, part)
            weight_map.update({n: file for n in part})
        # the map's own order: the second file named first
        ordered = dict(sorted(weight_map.items()))
        (root / "model.safetensors.index.json").write_text(
            json.dumps({"metadata": {"total_size": 1}, "weight_map": ordered}))
    else:
        write_shard(root / "model.safetensors", tensors)
    return root


def refused(gemma, directory, status=G.ERR_FORMAT):
    with pytest.raises(G.Gq8Error) as e:
        gemma.load(directory)
    assert e.value.status == status
    assert not gemma.is_loaded()
    return str(e.value)


def test_single_file_directory(tmp_path):
    shape = tiny_shape()
    root = model_directory(tmp_path / "m", shape, generation={"bos_token_id": 2, "eos_token_id": [7, 107],
                                                              "pad_token_id": None})
    g = G.Gemma()
    g.load(root)
    assert g.is_loaded() and not g.is_prepared()
    assert g.file(G.FILE_CONFIG) == str(root / "config.json")
    assert g.file(G.FILE_GENERATION_CONFIG) == str(root / "generation_config.json")
    assert g.file(G.FILE_TOKENIZER_JSON) == str(root / "tokenizer.json")
    # recorded only when present (ModelFiles.cpp:87-91)
    assert g.file(G.FILE_SHARD_INDEX) == "" and g.file(G.FILE_TOKENIZER_MODEL) == ""
    assert g.file(G.FILE_GGUF) == ""
    assert g.shards() == [str(root / "model.safetensors")]
    parsed, ids = g.config()
    assert (parsed.width, parsed.heads, parsed.kv_heads, parsed.head_dim, parsed.layers,
            parsed.intermediate, parsed.vocab, parsed.max_positions) == (
        128, 2, 1, 64, 2, 256, 1000, 64)
    # generation_config's eos (first of the list) over config.json's; a null
    # pad leaves config.json's
    assert ids == (2, 7, 0)


def test_sharded_directory_lists_shards_in_first_named_order(tmp_path):
    shape = tiny_shape()
    root = model_directory(tmp_path / "m", shape, sharded=True)
    g = G.Gemma()
    g.load(root)
    index = json.loads((root / "model.safetensors.index.json").read_text())["weight_map"]
    first_named = list(dict.fromkeys(index.values()))
    assert g.shards() == [str(root / f) for f in first_named]
    assert g.file(G.FILE_SHARD_INDEX) == str(root / "model.safetensors.index.json")
    assert g.config()[1] == (2, 1, 0)  # no generation_config.json


def test_required_files(tmp_path):
    shape = tiny_shape()
    g = G.Gemma()
    assert "is not a directory" in refused(g, tmp_path / "absent")
    root = model_directory(tmp_path / "noconfig", shape)
    (root / "config.json").unlink()
    assert "config.json" in refused(g, root)
    root = model_directory(tmp_path / "noweights", shape)
    (root / "model.safetensors").unlink()
    assert "model.safetensors" in refused(g, root)
    root = model_directory(tmp_path / "notokenizer", shape, tokenizer=False)
    assert "tokenizer.json" in refused(g, root)
    # a tokenizer naming more tokens than the embedding holds (Gemma.cpp:131-138)
    small = G.DecoderShape(128, 2, 1, 64, 2, 256, 160, 64, 16)
    root = model_directory(tmp_path / "smallvocab", small)
    assert "289" in refused(g, root)


def test_shard_index_refusals(tmp_path):
    shape = tiny_shape()
    g = G.Gemma()
    cases = {
        "missing": {"weight_map": {"model.norm.weight": "model-00009-of-00009.safetensors"}},
        "separator": {"weight_map": {"model.norm.weight": "../model.safetensors"}},
        "dotdot": {"weight_map": {"model.norm.weight": ".."}},
        "empty": {"weight_map": {}},
        "notobject": {"weight_map": ["model.safetensors"]},
        "notname": {"weight_map": {"model.norm.weight": 3}},
        "nomap": {"metadata": {}},
        "badmeta": {"weight_map": {"model.norm.weight": "model.safetensors"}, "metadata": 5},
    }
    messages = {}
    for name, index in cases.items():
        root = model_directory(tmp_path / name, shape)
        (root / "model.safetensors.index.json").write_text(json.dumps(index))
        messages[name] = refused(g, root)
    assert "model-00009-of-00009.safetensors" in messages["missing"]
    assert "not a plain file name" in messages["separator"]
    assert "not a plain file name" in messages["dotdot"]
    assert "names no shards" in messages["empty"]
    assert "not an object" in messages["notobject"]
    assert "not a file name" in messages["notname"]


def test_generation_config_refusals(tmp_path):
    shape = tiny_shape()
    g = G.Gemma()
    root = model_directory(tmp_path / "a", shape, generation={"eos_token_id": "one"})
    refused(g, root)
    root = model_directory(tmp_path / "b", shape)
    (root / "generation_config.json").write_text("[1, 2]")
    refused(g, root)
    # an empty list leaves config.json's id
    root = model_directory(tmp_path / "c", shape, generation={"eos_token_id": []})
    g.load(root)
    assert g.config()[1] == (2, 1, 0)


def test_settings_and_states(tmp_path, monkeypatch):
    shape = tiny_shape()
    g = G.Gemma()
    assert g.maximum_tokens == 0 and g.prompt_capacity == 512
    with pytest.raises(G.Gq8Error) as e:
        g.maximum_tokens = -1
    assert e.value.status == G.ERR_ARGUMENT
    with pytest.raises(G.Gq8Error) as e:
        g.prompt_capacity = 0
    assert e.value.status == G.ERR_ARGUMENT
    with pytest.raises(G.Gq8Error) as e:
        g.set_sampling(G.SamplingOptions(temperature=-1.0))
    assert e.value.status == G.ERR_ARGUMENT
    with pytest.raises(G.Gq8Error) as e:
        g.prepare()
    assert e.value.status == G.ERR_NOT_PREPARED
    with pytest.raises(G.Gq8Error) as e:
        g.text_for_tokens([5])
    assert e.value.status == G.ERR_NOT_PREPARED

    root = model_directory(tmp_path / "m", shape)
    g.maximum_tokens = 5
    g.prompt_capacity = 4
    g.load(root)
    assert g.maximum_tokens == 0  # load puts the limit back (Gemma.cpp:83)
    assert g.prompt_capacity == 4
    with pytest.raises(G.Gq8Error) as e:
        g.generate([2, 5])
    assert e.value.status == G.ERR_NOT_PREPARED
    with pytest.raises(G.Gq8Error) as e:
        g.generate_text("hello")
    assert e.value.status == G.ERR_NOT_PREPARED

    # textForTokens is the tokenizer's decode with the special tokens dropped
    tokenizer = G.Tokenizer.from_file(root / "tokenizer.json")
    ids = tokenizer.encode_with_bos("hello world")
    assert ids[0] == tokenizer.bos
    assert g.text_for_tokens(ids) == tokenizer.decode(ids)
    assert g.text_for_tokens(ids) == tokenizer.decode(ids[1:])

    monkeypatch.setenv("GEMMA_MODEL_DIR", str(root))
    assert G.model_directory_from_environment() == str(root)
    monkeypatch.setenv("GEMMA_MODEL_DIR", "")
    assert G.model_directory_from_environment() == ""
    monkeypatch.delenv("GEMMA_MODEL_DIR")
    assert G.model_directory_from_environment() == ""


def test_failed_load_leaves_nothing_loaded(tmp_path):
    shape = tiny_shape()
    g = G.Gemma()
    g.load(model_directory(tmp_path / "good", shape))
    assert g.is_loaded()
    bad = model_directory(tmp_path / "bad", shape)
    (bad / "model.safetensors").write_bytes(b"\x01\x00")
    refused(g, bad)
    assert g.shards() == []
