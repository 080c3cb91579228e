"""The benchmark configurations at their real sizes, against oracle fixtures
(tests/golden/gemma_*.npz, written by tests/golden/make_golden.py):

- the headline decode: 18 layers, 512-token prompt, 256 greedy tokens;
- the 2048-token prefill as one step of 2048 rows (int8 MFMA GEMMs, M = 2048);
- the long context: 18 layers, 8064-token prompt, decode to the end of the
  8192-position window;
- the same 18 layers with weight spreads under which the greedy ids change
  from step to step (the seeded N(0, 0.02) weights of the configurations
  repeat one id: a fixed point of the tied embedding).

What is held exactly: every greedy id, and the Q8 bytes of every layer's
product inputs (normalised, attended, activated) and of the final norm, as
SHA-256 digests of the oracle's bytes.  Logits: the metric's bar is 1e-2
relative (|a - e| / (1 + |e|)); the GPU and the oracle differ only in the
order of their double sums, so the tests also hold them to 1e-5 and print the
bit-identical fraction.  The reference's loop tests compare the same things
(Tests/Decoder/DecoderTests.cpp:96-180, Tests/Generation/GenerationTests.cpp:
192-224, 556-596; the tie gap of DecoderOracleTests.cpp:97-108 is the margin
printed here)."""
import hashlib
import os

import numpy as np
import pytest

import oracle as O
from gpu_helpers import empty, exact_fraction, to_device, worst_error
from huggingfaceeacp_amd import gemma_q8 as G

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LOGIT_TOLERANCE = 1e-2   # the metric's relative bar
SUM_ORDER_TOLERANCE = 1e-5
VARIED_SEED = 0x6A00


def fixture(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.skip(f"{name} not generated (python tests/golden/make_golden.py)")
    return np.load(path)


def step_logits(torch, decoder, tokens, logits_rows=1):
    tokens = np.asarray(tokens, dtype=np.uint32)
    ids = to_device(torch, tokens)
    if logits_rows == 0:
        decoder.step(ids.data_ptr(), tokens.size, None)
        torch.cuda.synchronize()
        return None
    logits = empty(torch, logits_rows * decoder.shape.vocab, torch.float32)
    decoder.step(ids.data_ptr(), tokens.size, logits.data_ptr(), logits_rows)
    torch.cuda.synchronize()
    return logits.cpu().numpy().reshape(logits_rows, decoder.shape.vocab)


def prefill(torch, decoder, tokens):
    """Steps of the decoder's capacity without logits."""
    capacity = decoder.shape.step_capacity()
    for start in range(0, len(tokens), capacity):
        step_logits(torch, decoder, tokens[start:start + capacity], 0)


def gpu_digests(decoder):
    """[layers + 1, 3, 32]: the SHA-256 of the last row's Q8 product inputs,
    laid out as the fixture's (tests/golden/make_golden.py q8_digests)."""
    layers = decoder.shape.layers
    out = np.zeros((layers + 1, 3, 32), np.uint8)
    for layer in range(layers):
        for which in range(3):
            _, q8 = decoder.debug(which, layer)
            out[layer, which] = np.frombuffer(hashlib.sha256(q8.tobytes()).digest(), np.uint8)
    _, q8 = decoder.debug(0, layers)
    out[layers, 0] = np.frombuffer(hashlib.sha256(q8.tobytes()).digest(), np.uint8)
    return out


def assert_digests(got, expected, label):
    differing = [(layer, which) for layer in range(expected.shape[0]) for which in range(3)
                 if not np.array_equal(got[layer, which], expected[layer, which])]
    print(f"  {label}: Q8 digests differing from the oracle's: {differing}")
    assert not differing, label


def check_row(row, top_ids, top_logits, label):
    err = worst_error(row[top_ids], top_logits)
    assert int(np.argmax(row)) == int(top_ids[0]), label
    assert err <= LOGIT_TOLERANCE, (label, err)
    assert err <= SUM_ORDER_TOLERANCE, (label, err)
    return exact_fraction(row[top_ids], top_logits)


def stepwise(torch, decoder, f, digest_steps=()):
    """The fixture's loop a step at a time on the GPU: the prompt (the last
    row as a one-row step, debug on), then one step per id, each step's
    top-8 logits against the fixture's; the Q8 digests where it has them."""
    prompt, ids = f["prompt"], f["ids"]
    decoder.begin_sequence()
    prefill(torch, decoder, prompt[:-1])
    decoder.set_debug(True)
    row = step_logits(torch, decoder, prompt[-1:])[0]
    assert_digests(gpu_digests(decoder), f["digests"][0], "last prompt row")
    decoder.set_debug(False)
    assert worst_error(row[::1000], f["prompt_row_every_1000th"]) <= SUM_ORDER_TOLERANCE
    exact = []
    for s in range(len(ids)):
        exact.append(check_row(row, f["top_ids"][s], f["top_logits"][s], f"step {s}"))
        if s + 1 == len(ids):
            break
        debug_here = (s + 1) in digest_steps
        decoder.set_debug(debug_here)
        row = step_logits(torch, decoder, [int(ids[s])])[0]
        if debug_here:
            k = list(digest_steps).index(s + 1) + 1
            assert_digests(gpu_digests(decoder), f["digests"][k], f"generated step {s + 1}")
    decoder.set_debug(False)
    return float(np.mean(exact))


def test_config2_headline_512_plus_256(torch_cuda):
    """18 layers, the 512-token prompt, 256 greedy tokens: the plain loop and
    the graph replay give the oracle's ids; every step's top-8 logits and the
    last prompt row's Q8 bytes are the oracle's."""
    torch = torch_cuda
    f = fixture("gemma_ctx512.npz")
    print("config 2: 18 layers, 512 + 256", flush=True)
    shape = G.DecoderShape.gemma_2b(layers=18, max_positions=1024, max_step_rows=512)
    decoder = G.Decoder(shape)
    decoder.fill_synthetic(16)
    expected = list(f["ids"])
    assert decoder.attention_path == 1
    for label, graph in (("graph", True), ("plain", False)):
        tokens, stats = decoder.generate(f["prompt"], 256, eos=-1, use_graph=graph)
        print(f"  {label}: {len(tokens)} ids, decode {stats.decode_seconds * 1e3:.1f} ms", flush=True)
        assert list(tokens) == expected, label
    exact = stepwise(torch, decoder, f)
    print(f"  top-8 logits bit-identical in {exact:.4f} of places; smallest top-2 margin "
          f"{f['margins'].min():.3g}; distinct ids {len(set(expected))}")


def test_config3_prefill_2048_rows(torch_cuda):
    """One 2048-row step at 18 layers (every product an int8 MFMA GEMM of
    M = 2048): the last row's logits and the Q8 bytes of rows 0, 1023 and
    2047 are the oracle's, and the rows equal the one-row kernels' (a row
    computed inside a block is the row computed alone)."""
    torch = torch_cuda
    f = fixture("gemma_prefill2048.npz")
    print("config 3: one 2048-row step, 18 layers", flush=True)
    prompt = f["prompt"]
    shape = G.DecoderShape.gemma_2b(layers=18, max_positions=2048, max_step_rows=2048)
    decoder = G.Decoder(shape)
    decoder.fill_synthetic(16)
    decoder.set_debug(True)
    block = step_logits(torch, decoder, prompt, 1)[0]
    assert_digests(gpu_digests(decoder), f["digests"][2], "row 2047 of the 2048-row step")
    exact = check_row(block, f["top_ids"], f["top_logits"], "last row")
    assert worst_error(block[::1000], f["every_1000th"]) <= SUM_ORDER_TOLERANCE
    print(f"  last-row top-64 logits bit-identical in {exact:.4f} of places", flush=True)

    # row 0 alone (the one-row kernels), row 1023 as the last of a 1024-row step
    decoder.begin_sequence()
    step_logits(torch, decoder, prompt[:1], 1)
    assert_digests(gpu_digests(decoder), f["digests"][0], "row 0, one-row step")
    decoder.begin_sequence()
    step_logits(torch, decoder, prompt[:1024], 1)
    assert_digests(gpu_digests(decoder), f["digests"][1], "row 1023, 1024-row step")
    # rows 1023 and 2047 by the one-row kernels after a multi-row prefix
    decoder.begin_sequence()
    decoder.set_debug(False)
    step_logits(torch, decoder, prompt[:1023], 0)
    decoder.set_debug(True)
    step_logits(torch, decoder, prompt[1023:1024], 1)
    assert_digests(gpu_digests(decoder), f["digests"][1], "row 1023, one-row step")
    decoder.set_debug(False)
    step_logits(torch, decoder, prompt[1024:2047], 0)
    decoder.set_debug(True)
    alone = step_logits(torch, decoder, prompt[2047:], 1)[0]
    assert_digests(gpu_digests(decoder), f["digests"][2], "row 2047, one-row step")
    decoder.set_debug(False)
    err = worst_error(alone, block)
    print(f"  row 2047 alone vs in the block: worst {err:.3g}, exact {exact_fraction(alone, block):.4f}")
    assert err <= SUM_ORDER_TOLERANCE


def test_config4_long_context_18_layers(torch_cuda):
    """18 layers, the 8064-token prompt, greedy decode to the end of the
    8192-position window: the oracle's 128 ids (graph replay and plain loop),
    every step's top-8 logits, and the window's refusal past its end."""
    torch = torch_cuda
    f = fixture("gemma_long8192.npz")
    print("config 4: 18 layers, 8064 + 128", flush=True)
    shape = G.DecoderShape.gemma_2b(layers=18, max_positions=8192, max_step_rows=512)
    decoder = G.Decoder(shape)
    decoder.fill_synthetic(16)
    expected = list(f["ids"])
    for label, graph in (("graph", True), ("plain", False)):
        tokens, stats = decoder.generate(f["prompt"], 1000, eos=-1, use_graph=graph)
        print(f"  {label}: {len(tokens)} ids, decode {stats.decode_seconds * 1e3:.1f} ms", flush=True)
        assert list(tokens) == expected, label
    assert decoder.position == 8191
    decoder.decode(1)
    with pytest.raises(G.Gq8Error) as e:
        decoder.decode(1)
    assert e.value.status == G.ERR_WINDOW
    exact = stepwise(torch, decoder, f)
    print(f"  top-8 logits bit-identical in {exact:.4f} of places")


def varied_decoder(layers, max_positions, max_step_rows=64):
    shape = G.DecoderShape.gemma_2b(layers=layers, max_positions=max_positions,
                                    max_step_rows=max_step_rows)
    decoder = G.Decoder(shape)
    for index in range(shape.tensor_count()):
        values = G.normal_fill_host(VARIED_SEED + index, varied_sigma(shape, index),
                                    shape.tensor_elements(index))
        decoder.load_tensor(index, values)
    return shape, decoder


def varied_sigma(shape, index):
    """Embedding 0.02, norms 0.1, projections 3 / sqrt(fan in)."""
    if index == 0:
        return 0.02
    if shape.tensor_is_norm(index):
        return 0.1
    role = (index - 1) % G.PER_LAYER
    fan_in = {G.T_O: shape.query_width, G.T_DOWN: shape.intermediate}.get(role, shape.width)
    return 3.0 / np.sqrt(fan_in)


def test_varied_ids_18_layers(torch_cuda):
    """18 layers at Gemma-2B dims with ids that change every step: the
    oracle's 48 ids on every decode path, each step's top-8 logits, and the
    Q8 bytes of every layer at the last prompt row and at step 24."""
    torch = torch_cuda
    f = fixture("gemma_varied18.npz")
    print("varied spreads: 18 layers, 64 + 48", flush=True)
    shape, decoder = varied_decoder(18, 256)
    expected = list(f["ids"])
    assert len(set(expected)) > 40
    for label, graph, fused in (("graph", True, True), ("plain", False, True),
                                ("unfused", False, False)):
        decoder.set_fused(fused)
        tokens, _ = decoder.generate(f["prompt"], 48, eos=-1, use_graph=graph)
        assert list(tokens) == expected, label
    decoder.set_fused(True)
    exact = stepwise(torch, decoder, f, digest_steps=tuple(int(s) for s in f["digest_steps"]))
    print(f"  distinct ids {len(set(expected))}, smallest top-2 margin {f['margins'].min():.3g}, "
          f"top-8 logits bit-identical in {exact:.4f} of places")


def test_varied_ids_18_layers_past_512_keys(torch_cuda):
    """The same weights past 512 keys, where a step's attention is the
    launch of 513-1024 keys (32 splits): the oracle's 24 ids through the
    graph and the plain loop, each step's top-8 logits, and every layer's Q8
    bytes at the last prompt row (560 keys) and at generated steps 1, 12
    and 23 (561, 572 and 583 keys)."""
    torch = torch_cuda
    f = fixture("gemma_varied18_ctx560.npz")
    print("varied spreads: 18 layers, 560 + 24", flush=True)
    shape, decoder = varied_decoder(18, 1024)
    expected = list(f["ids"])
    assert len(set(expected)) > 16
    for label, graph in (("graph", True), ("plain", False)):
        tokens, _ = decoder.generate(f["prompt"], len(expected), eos=-1, use_graph=graph)
        assert list(tokens) == expected, label
    exact = stepwise(torch, decoder, f, digest_steps=tuple(int(s) for s in f["digest_steps"]))
    print(f"  distinct ids {len(set(expected))}, smallest top-2 margin {f['margins'].min():.3g}, "
          f"top-8 logits bit-identical in {exact:.4f} of places")


def test_varied_ids_two_layers_q8_bytes(torch_cuda):
    """2 layers, the same spreads, against the live oracle: every Q8 byte of
    every layer's product inputs (counted, not hashed), the ids and logits."""
    torch = torch_cuda
    shape, decoder = varied_decoder(2, 128)
    model = O.Model(O.gemma_2b_shape(layers=2, max_positions=128), O.MODE_Q8)
    for index in range(shape.tensor_count()):
        values = O.normal_fill(VARIED_SEED + index, varied_sigma(shape, index),
                               shape.tensor_elements(index))
        assert model.set_tensor(index, values) == 0
    prompt = O.prompt_ids(0xC0FFEE + 8, shape.vocab, 24)
    tokens, _ = decoder.generate(prompt, 24, eos=-1)
    _, ref_ids, margins = model.generate(prompt, 24, eos=-1)
    print(f"2-layer varied: ids {list(tokens)[:8]}..., distinct {len(set(tokens))}, "
          f"smallest margin {margins.min():.3g}")
    assert list(tokens) == list(ref_ids)
    assert len(set(tokens)) > 16
    # the Q8 bytes of the last prompt row and of the first three decode steps
    decoder.begin_sequence()
    model.begin()
    prefill(torch, decoder, prompt[:-1])
    assert model.step(prompt[:-1], want_logits=False)[0] == 0
    inner = {0: shape.width, 1: shape.query_width, 2: shape.intermediate}
    feed = [int(prompt[-1])] + [int(t) for t in ref_ids[:3]]
    for k, token in enumerate(feed):
        decoder.set_debug(True)
        row = step_logits(torch, decoder, [token])[0]
        _, ref, _ = model.step(np.array([token], np.int32))
        mismatched = 0
        for layer in range(shape.layers + 1):
            for which in ((0, 1, 2) if layer < shape.layers else (0,)):
                _, q8 = decoder.debug(which, layer)
                rq, rs = model.debug_q(which, layer)
                n = inner[which]
                mismatched += int(np.sum(q8[:n].view(np.int8) != rq))
                mismatched += int(np.sum(q8[n:].view(np.uint16) != rs))
        err = worst_error(row, ref[0])
        print(f"  step {k}: Q8 bytes differing {mismatched}, logits worst {err:.3g}, "
              f"exact {exact_fraction(row, ref[0]):.4f}")
        assert mismatched == 0
        assert err <= SUM_ORDER_TOLERANCE
    decoder.set_debug(False)
