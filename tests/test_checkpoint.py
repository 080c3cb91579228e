"""Checkpoint files on the host: safetensors headers and widening, and Gemma's
config.json, through the C ABI (no GPU needed).

The cases restate the reference's own tests (Tests/Model/SafeTensorsTests.cpp,
Tests/Model/ConfigTests.cpp) on files assembled here byte for byte.  The
widening is checked against definitions, not against this code: a bfloat16
is the top 16 bits of a float32, and half precision is numpy's IEEE binary16.
"""
import dataclasses
import json
import struct

import numpy as np
import pytest

from huggingfaceeacp_amd import gemma_q8 as G


def assemble(header, blob=b"", declared=None):
    """8-byte little-endian header length, the header, the blob."""
    text = header if isinstance(header, bytes) else header.encode()
    length = len(text) if declared is None else declared
    return struct.pack("<Q", length) + text + blob


SINGLE = '{"weight":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]}}'


def single_file():
    return assemble(SINGLE, np.arange(1, 7, dtype=np.float32).tobytes())


def refused(make, status=G.ERR_FORMAT):
    with pytest.raises(G.Gq8Error) as e:
        make()
    assert e.value.status == status, str(e.value)


def test_single_tensor():
    f = G.SafeTensors.from_bytes(single_file())
    assert f.names() == ["weight"]
    assert f.info("weight") == ("F32", (2, 3), 24)
    assert np.array_equal(f.read_floats("weight"), np.arange(1, 7, dtype=np.float32))
    assert f.metadata() == {}


def test_float_round_trips():
    values = np.array([0.0, -0.0, 1.5, -2.25, 3.4028235e38, 1e-45, np.inf, -np.inf], np.float32)
    f = G.SafeTensors.from_bytes(assemble(
        '{"x":{"dtype":"F32","shape":[8],"data_offsets":[0,32]}}', values.tobytes()))
    assert f.read_floats("x").tobytes() == values.tobytes()


# Every class bfloat16 has: zeros, subnormals, one, ordinary magnitudes, the
# largest finite value, both infinities, quiet and signalling NaNs.
BFLOAT_SWEEP = [0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x0080, 0x3F80, 0xBF80, 0x4049, 0x3EAA,
                0xC2F0, 0x7F7F, 0xFF7F, 0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x0002, 0x00FF, 0x4780]


def test_bfloat_widens_exactly():
    bits = np.array(BFLOAT_SWEEP, dtype=np.uint16)
    header = '{"b":{"dtype":"BF16","shape":[%d],"data_offsets":[0,%d]}}' % (bits.size, 2 * bits.size)
    f = G.SafeTensors.from_bytes(assemble(header, bits.tobytes()))
    got = f.read_floats("b").view(np.uint32)
    assert np.array_equal(got, bits.astype(np.uint32) << 16)


def test_half_widens_to_float():
    halves = np.array([0.0, -0.0, 1.0, -2.5, 65504.0, 6e-8, 6.1035156e-05, np.inf, -np.inf],
                      dtype=np.float16)
    header = '{"h":{"dtype":"F16","shape":[%d],"data_offsets":[0,%d]}}' % (halves.size, 2 * halves.size)
    f = G.SafeTensors.from_bytes(assemble(header, halves.tobytes()))
    assert np.array_equal(f.read_floats("h"), halves.astype(np.float32))
    # every finite half through the same widening
    every = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    every = every[np.isfinite(every.view(np.float16))]
    header = '{"h":{"dtype":"F16","shape":[%d],"data_offsets":[0,%d]}}' % (every.size, 2 * every.size)
    f = G.SafeTensors.from_bytes(assemble(header, every.tobytes()))
    assert np.array_equal(f.read_floats("h"), every.view(np.float16).astype(np.float32))


def test_read_into_destination():
    f = G.SafeTensors.from_bytes(single_file())
    assert np.array_equal(f.read_floats("weight", 2, 3), np.array([3, 4, 5], np.float32))
    assert f.read_floats("weight", 6, 0).size == 0
    refused(lambda: f.read_floats("weight", 4, 3), G.ERR_ARGUMENT)


def test_multiple_tensors_and_metadata():
    header = json.dumps({
        "__metadata__": {"format": "pt", "origin": "here"},
        "zeta": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},
        "alpha": {"dtype": "BF16", "shape": [2], "data_offsets": [4, 8]},
    })
    blob = np.float32(7.0).tobytes() + np.array([0x3F80, 0x4000], np.uint16).tobytes()
    f = G.SafeTensors.from_bytes(assemble(header, blob))
    assert f.names() == ["alpha", "zeta"]  # sorted by name
    assert f.metadata() == {"format": "pt", "origin": "here"}
    assert np.array_equal(f.read_floats("alpha"), np.array([1.0, 2.0], np.float32))
    assert f.read_floats("zeta")[0] == 7.0
    assert f.raw("alpha") == blob[4:8]


def test_integer_tensors_are_not_floats():
    f = G.SafeTensors.from_bytes(assemble(
        '{"w":{"dtype":"I32","shape":[2],"data_offsets":[0,8]}}', struct.pack("<ii", 1, 2)))
    assert f.info("w") == ("I32", (2,), 8)
    assert len(f.raw("w")) == 8
    refused(lambda: f.read_floats("w"))


def test_unknown_tensor_lookup():
    f = G.SafeTensors.from_bytes(single_file())
    assert not f.contains("nope")
    refused(lambda: f.info("nope"))
    refused(lambda: f.raw("nope"))


def test_malformed_headers():
    refused(lambda: G.SafeTensors.from_bytes(b"\0" * 7))
    refused(lambda: G.SafeTensors.from_bytes(assemble("{}", declared=3)))
    refused(lambda: G.SafeTensors.from_bytes(assemble("{}", declared=(1 << 64) - 1)))
    for header in ["{not json", "[1,2,3]", "", '{"w":42}']:
        refused(lambda: G.SafeTensors.from_bytes(assemble(header)))


def test_missing_fields():
    for header in ['{"w":{"shape":[1],"data_offsets":[0,4]}}',
                   '{"w":{"dtype":"F32","data_offsets":[0,4]}}',
                   '{"w":{"dtype":"F32","shape":[1]}}',
                   '{"w":{"dtype":"F8_E4M3","shape":[1],"data_offsets":[0,1]}}']:
        refused(lambda: G.SafeTensors.from_bytes(assemble(header, b"\0" * 4)))


def test_shape_disagrees_with_range():
    blob = np.array([1.0, 2.0], np.float32).tobytes()
    for header in ['{"w":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}',
                   '{"w":{"dtype":"BF16","shape":[2],"data_offsets":[0,8]}}',
                   '{"w":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}',
                   '{"w":{"dtype":"F32","shape":[1],"data_offsets":[8,4]}}',
                   '{"w":{"dtype":"F32","shape":[-1],"data_offsets":[0,0]}}']:
        refused(lambda: G.SafeTensors.from_bytes(assemble(header, blob)))


def test_metadata_must_be_strings():
    refused(lambda: G.SafeTensors.from_bytes(assemble('{"__metadata__":{"format":7}}')))
    refused(lambda: G.SafeTensors.from_bytes(assemble('{"__metadata__":7}')))


def test_empty_tensor_is_legal():
    f = G.SafeTensors.from_bytes(assemble('{"empty":{"dtype":"F32","shape":[0,4],"data_offsets":[0,0]}}'))
    assert f.info("empty") == ("F32", (0, 4), 0)
    assert f.read_floats("empty").size == 0


def test_missing_file_is_an_error(tmp_path):
    refused(lambda: G.SafeTensors.open("no/such/model.safetensors"))
    refused(lambda: G.SafeTensors.open(tmp_path))


def test_mapped_file_matches_bytes(tmp_path):
    path = tmp_path / "model.safetensors"
    path.write_bytes(single_file())
    mapped = G.SafeTensors.open(path)
    in_memory = G.SafeTensors.from_bytes(single_file())
    assert mapped.names() == in_memory.names()
    assert mapped.info("weight") == in_memory.info("weight")
    assert np.array_equal(mapped.read_floats("weight"), in_memory.read_floats("weight"))


# ---- config.json (Tests/Model/ConfigTests.cpp) ----------------------------------------
def gemma_config_json(overrides=""):
    # overrides first: the first occurrence of a duplicate key wins
    return ("{" + (overrides + "," if overrides else "")
            + '"model_type":"gemma","vocab_size":256000,"hidden_size":2048,'
              '"intermediate_size":16384,"num_hidden_layers":18,"num_attention_heads":8,'
              '"num_key_value_heads":1,"head_dim":256,"max_position_embeddings":8192,'
              '"rms_norm_eps":1e-06,"rope_theta":10000.0,"hidden_activation":"gelu_pytorch_tanh",'
              '"bos_token_id":2,"eos_token_id":1,"pad_token_id":0,"tie_word_embeddings":true}')


def test_config_shapes():
    shape, ids = G.gemma_config(gemma_config_json(), max_step_rows=512)
    assert np.float32(shape.rms_epsilon) == np.float32(1e-6)  # carried as the fp32 eps
    assert dataclasses.replace(shape, rms_epsilon=1e-6) == G.DecoderShape.gemma_2b(18, 8192, 512)
    assert ids == (2, 1, 0)
    assert shape.query_width == 2048 and shape.kv_width == 256
    assert abs(shape.embedding_scale - 45.254834) < 1e-4


def test_config_defaults_and_window():
    full, ids = G.gemma_config(gemma_config_json())
    assert G.gemma_config('{"model_type":"gemma"}') == (full, ids)
    assert G.gemma_config("{}")[0].width == 2048
    # a caller's window below max_position_embeddings
    assert G.gemma_config(gemma_config_json(), max_positions=1024)[0].max_positions == 1024
    # eos as a list takes the first entry; null keeps the default
    assert G.gemma_config('{"eos_token_id":[107,1]}')[1] == (2, 107, 0)
    assert G.gemma_config('{"eos_token_id":null}')[1] == (2, 1, 0)


def test_config_rejects_another_architecture():
    refused(lambda: G.gemma_config('{"model_type":"llama"}'))
    refused(lambda: G.gemma_config(gemma_config_json('"model_type":"t5"')))


def test_config_rejects_bad_shapes():
    for text in ["not json", "[]"]:
        refused(lambda: G.gemma_config(text))
    for override in ['"hidden_size":0', '"num_hidden_layers":-1', '"rms_norm_eps":0',
                     '"rope_theta":-1', '"hidden_size":"2048"', '"hidden_size":2048.5',
                     '"num_attention_heads":3,"num_key_value_heads":2']:
        refused(lambda: G.gemma_config(gemma_config_json(override)))
    # this decoder's lm_head is the embedding
    refused(lambda: G.gemma_config(gemma_config_json('"tie_word_embeddings":false')), G.ERR_SHAPE)
