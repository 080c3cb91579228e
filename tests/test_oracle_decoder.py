"""Pins of the oracle's whole decoder (CPU only).

  - Its reference mode (the double chain of Tests/Decoder/ReferenceDecoder.h)
    against an independent implementation of Gemma: transformers'
    GemmaForCausalLM in float64, with the same dequantized weights.  The two
    differ only where the reference fixes fp32 constants (the fp32 rotary
    table, the embedding scale 45.254833f, epsilon 1e-6f), within the
    reference's own decoder tolerance of 5e-6 (DecoderTests.cpp:41-180).
  - Its Q8 path with the two storage rules off (fp32 product inputs, an fp32
    KV cache) against the reference mode, at the same tolerance: the
    composition of the path's code.
  - Its Q8 path against the reference mode at the Gemma shape: logits within
    1e-2 of the row's largest and the same greedy ids.
  - The reference's own decoder equivalences: a prompt in one step, one
    token at a time and in two blocks give the same bits (DecoderTests.cpp:
    116-147, 418-463); the greedy loop stops at EOS and at the window
    (GenerationTests.cpp:192-224, Gemma.cpp:395-543).
"""
import numpy as np
import pytest

import oracle as O

PROMPT = [5, 41, 3, 17, 28, 9, 60]  # Tests/Decoder/DecoderTests.cpp:41-60


def small_shape(max_positions=16):
    # Tests/Decoder/Common.h:38-72, the quantizable variant (FFN 64)
    return O.make_shape(32, 2, 1, 16, 2, 64, 64, max_positions)


def small_tensors(probe):
    """N(0, 0.2) projections and embedding, N(0, 0.1) norms, seeded per tensor."""
    return [O.normal_fill(0x7100 + i, 0.1 if probe.is_norm(i) else 0.2, probe.tensor_elements(i))
            for i in range(probe.tensor_count)]


def build(shape, mode, values):
    model = O.Model(shape, mode)
    for i, v in enumerate(values):
        assert model.set_tensor(i, v) == 0
    return model


@pytest.fixture(scope="module")
def small():
    shape = small_shape()
    probe = O.Model(shape, O.MODE_Q8)
    values = small_tensors(probe)
    probe.close()
    return shape, values


def worst_relative(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b) / (1.0 + np.abs(b))))


def test_reference_mode_matches_transformers_gemma_in_float64(small):
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    shape, values = small
    ref = build(shape, O.MODE_REFERENCE, values)

    def weight(i, rows, cols):
        if ref.is_norm(i):
            return torch.tensor(values[i].astype(np.float64))
        recovered = O.dequantize_int8_blocks(ref.tensor_bytes(i), ref.tensor_elements(i))
        return torch.tensor(recovered.astype(np.float64).reshape(rows, cols))

    config = transformers.GemmaConfig(
        vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
        num_attention_heads=2, num_key_value_heads=1, head_dim=16, max_position_embeddings=16,
        rms_norm_eps=1e-6, rope_theta=10000.0, hidden_activation="gelu_pytorch_tanh",
        tie_word_embeddings=True)
    torch.manual_seed(0)
    hf = transformers.GemmaForCausalLM(config).double().eval()
    state = {"model.embed_tokens.weight": weight(0, 64, 32), "model.norm.weight": weight(19, 0, 0)}
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
             "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    shapes = [(32, 32), (16, 32), (16, 32), (32, 32), (64, 32), (64, 32), (32, 64)]
    for layer in range(2):
        base = 1 + 9 * layer
        for j, (name, (rows, cols)) in enumerate(zip(names, shapes)):
            state[f"model.layers.{layer}.{name}.weight"] = weight(base + j, rows, cols)
        state[f"model.layers.{layer}.input_layernorm.weight"] = weight(base + 7, 0, 0)
        state[f"model.layers.{layer}.post_attention_layernorm.weight"] = weight(base + 8, 0, 0)
    state["lm_head.weight"] = state["model.embed_tokens.weight"]
    hf.load_state_dict(state, strict=False)
    with torch.no_grad():
        theirs = hf(torch.tensor([PROMPT]), use_cache=False).logits[0].numpy()
    status, ours, _ = ref.step(np.array(PROMPT))
    assert status == 0
    assert worst_relative(ours, theirs) < 5e-6


def test_q8_path_code_without_the_storage_rules_matches_the_reference(small):
    shape, values = small
    ref = build(shape, O.MODE_REFERENCE, values)
    path = build(shape, O.MODE_Q8_PATH_F32, values)
    _, want, _ = ref.step(np.array(PROMPT))
    _, got, _ = path.step(np.array(PROMPT))
    assert worst_relative(got, want) < 5e-6
    # and the decode steps after it
    for token in (7, 30, 2):
        _, want, _ = ref.step(np.array([token]))
        _, got, _ = path.step(np.array([token]))
        assert worst_relative(got, want) < 5e-6


def test_prompt_in_one_step_token_by_token_and_in_two_blocks_agree(small):
    shape, values = small
    whole = build(shape, O.MODE_Q8, values)
    _, once, _ = whole.step(np.array(PROMPT))
    single = build(shape, O.MODE_Q8, values)
    rows = [single.step(np.array([t]))[1][0] for t in PROMPT]
    assert np.array_equal(np.stack(rows), once)
    blocks = build(shape, O.MODE_Q8, values)
    first = blocks.step(np.array(PROMPT[:3]))[1]
    second = blocks.step(np.array(PROMPT[3:]))[1]
    assert np.array_equal(np.concatenate([first, second]), once)


def test_greedy_loop_is_the_argmax_loop_with_eos_and_window(small):
    shape, values = small
    looped = build(shape, O.MODE_Q8, values)
    count, ids, _ = looped.generate(np.array(PROMPT), 9, eos=-1)
    assert count == shape.max_positions - len(PROMPT)  # the window limit, 16 - 7
    manual = build(shape, O.MODE_Q8, values)
    _, logits, _ = manual.step(np.array(PROMPT))
    token = O.argmax(logits[-1])
    want = []
    for _ in range(count):
        want.append(token)
        _, logits, _ = manual.step(np.array([token]))
        token = O.argmax(logits[0])
    assert list(ids) == want
    # an EOS id stops the loop and is not emitted
    stopper = build(shape, O.MODE_Q8, values)
    eos = int(ids[2])
    count, got, _ = stopper.generate(np.array(PROMPT), 9, eos=eos)
    assert list(got) == list(ids[:list(ids).index(eos)])


@pytest.mark.slow
def test_q8_path_is_within_one_percent_of_the_reference_at_the_gemma_shape():
    # the two-layer Gemma workload: seeded N(0, 0.02) weights, N(0, 0.1) norms,
    # a 16-token seeded prompt
    shape = O.gemma_2b_shape(layers=2, max_positions=64)
    q8 = O.Model(shape, O.MODE_Q8)
    ref = O.Model(shape, O.MODE_REFERENCE)
    assert q8.fill_synthetic() == 0 and ref.fill_synthetic() == 0
    prompt = O.prompt_ids(0xC0FFEE + 1, shape.vocab, 16)
    _, got, _ = q8.step(prompt)
    _, want, _ = ref.step(prompt)
    for row in range(16):
        scale = float(np.max(np.abs(want[row])))
        assert float(np.max(np.abs(got[row] - want[row]))) <= 1e-2 * scale
        assert int(np.argmax(got[row])) == int(np.argmax(want[row]))


@pytest.mark.parametrize("gemma", [False, True])
def test_block_step_is_bit_identical_to_single_steps(small, gemma):
    """The oracle's blocked prefill (products over all rows of a block at
    once) against token-at-a-time steps: the same logits and Q8 activation
    bytes, bit for bit, including across the block boundary of 256 rows."""
    if gemma:
        shape = O.gemma_2b_shape(layers=1, max_positions=320)
        prompt = O.prompt_ids(0xC0FFEE + 11, shape.vocab, 300)
        one, block = O.Model(shape, O.MODE_Q8), O.Model(shape, O.MODE_Q8)
        assert one.fill_synthetic() == 0 and block.fill_synthetic() == 0
    else:
        shape, values = small
        prompt = np.array(PROMPT * 2, dtype=np.int32)
        one, block = build(shape, O.MODE_Q8, values), build(shape, O.MODE_Q8, values)
    assert one.step(prompt[:-1], want_logits=False)[0] == 0
    status, want, _ = one.step(prompt[-1:])
    assert status == 0
    status, got = block.step_block(prompt, logits_rows=1)
    assert status == 0
    assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
    assert block.position == one.position == prompt.size
    for layer in range(shape.layers):
        for which in (O.DBG_NORMALISED, O.DBG_ATTENDED, O.DBG_ACTIVATED):
            for a, b in zip(block.debug_q(which, layer), one.debug_q(which, layer)):
                assert np.array_equal(a, b), (layer, which)
    # and the next single step continues from the block's cache exactly
    token = np.array([int(np.argmax(want[0]))], dtype=np.int32)
    assert np.array_equal(block.step(token)[1][0].view(np.uint32), one.step(token)[1][0].view(np.uint32))
