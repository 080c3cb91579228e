"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

The reference commits no numeric fixtures of its own (its tests compute their
expectations from mt19937-seeded inputs), so these are the oracle's outputs on
seeded inputs, committed so that the GPU tests and later changes to the oracle
are held to fixed bytes:

  int8_blocks.npz   Int8Blocks encodings of blocks chosen for the rounding
                    rule: near-ties, subnormal and overflowing scales, zeros;
  rotary.npz        rotary table rows (head_dim 256) at positions 0, 1, 8191;
  small_model.npz   the small test model (width 32, 2 heads / 1 KV head of 16,
                    2 layers, FFN 64, vocabulary 64) on the prompt
                    {5, 41, 3, 17, 28, 9, 60}: Q8-path and reference logits;
  two_layer_gemma.npz  the two-layer Gemma workload (seeded N(0, 0.02)
                    weights, N(0, 0.1) norms, 16-token seeded prompt): the
                    Q8 path's 32 greedy ids, each step's top-8 ids and logits,
                    and every 1000th logit of the last prompt row.

The full-size fixtures take minutes of CPU each and are written on request
(`python tests/golden/make_golden.py ctx512 prefill2048 varied18 varied18_ctx560
long8192`):

  gemma_ctx512.npz  18 layers, seeded N(0, 0.02) weights, the 512-token
                    prompt of seed 0xC0FFEE + 2, 256 greedy tokens (no EOS
                    stop): ids, per-step top-8 ids and logits, top-2 margins,
                    and the SHA-256 of every layer's Q8 product inputs
                    (normalised, attended, activated) and the final norm's Q8
                    row for the last prompt row;
  gemma_prefill2048.npz  18 layers, the 2048-token prompt of seed 0xC0FFEE + 3:
                    the last row's top-64 ids and logits, every 1000th logit,
                    and the Q8 digests of rows 0, 1023 and 2047;
  gemma_varied18.npz  18 layers with spreads under which the greedy ids change
                    from step to step (embedding 0.02, norms 0.1, projections
                    3 / sqrt(fan in), tensor seeds 0x6A00 + index), the
                    64-token prompt of seed 0xC0FFEE + 7, 48 greedy tokens:
                    ids, top-8 ids and logits, margins, and the Q8 digests of
                    the last prompt row and of the 24th generated step;
  gemma_varied18_ctx560.npz  the same weights past 512 keys: the 560-token
                    prompt of seed 0xC0FFEE + 9, 24 greedy tokens, with the Q8
                    digests of the last prompt row and of generated steps 1,
                    12 and 23 (561, 572 and 583 keys);
  gemma_long8192.npz  18 layers, seeded N(0, 0.02) weights, the 8064-token
                    prompt of seed 0xC0FFEE + 4, greedy decode to the end of
                    the 8192-position window (128 ids): ids, top-8 ids and
                    logits, margins.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

PROMPT = [5, 41, 3, 17, 28, 9, 60]


def int8_block_inputs():
    rng = np.random.default_rng(20250101)
    blocks = []
    for scale_exp in (-26, -20, -14, -8, -2, 0, 4, 9):
        scale = np.float32(np.float16(np.float32(2.0 ** scale_exp * 1.37)))
        k = rng.integers(-127, 127, 32)
        ties = ((k + 0.5) * np.float64(scale)).astype(np.float32)
        ties[0] = np.float32(127 * np.float64(scale))  # the amax, so the scale is as chosen
        nudged = ties.copy()
        nudged[1::2] = np.nextafter(nudged[1::2], np.float32(np.inf))
        blocks += [ties, nudged]
    blocks.append(np.zeros(32, np.float32))
    blocks.append(np.full(32, 6.0e-8, np.float32))                 # scale below fp16
    blocks.append(np.full(32, 65504.0 * 127 * 2, np.float32))      # scale above fp16
    blocks.append((rng.standard_normal(32) * 0.02).astype(np.float32))
    blocks.append((rng.standard_normal(32) * 3.0).astype(np.float32))
    return np.concatenate(blocks)


def small_model():
    shape = O.make_shape(32, 2, 1, 16, 2, 64, 64, 16)
    out = {}
    for name, mode in (("q8", O.MODE_Q8), ("reference", O.MODE_REFERENCE)):
        model = O.Model(shape, mode)
        for i in range(model.tensor_count):
            sigma = 0.1 if model.is_norm(i) else 0.2
            assert model.set_tensor(i, O.normal_fill(0x7100 + i, sigma, model.tensor_elements(i))) == 0
        status, logits, _ = model.step(np.array(PROMPT))
        assert status == 0
        out[f"{name}_logits"] = logits
        model.close()
    return out


def top(logits, count):
    order = np.argsort(-logits.astype(np.float64), kind="stable")[:count]
    return order.astype(np.int32), logits[order]


def two_layer_gemma():
    """The prompt step and 31 decode steps by hand (the greedy loop), keeping
    each step's top-8 ids and logits and a strided sample of the prompt row."""
    shape = O.gemma_2b_shape(layers=2, max_positions=64)
    model = O.Model(shape, O.MODE_Q8)
    assert model.fill_synthetic() == 0
    prompt = O.prompt_ids(0xC0FFEE + 1, shape.vocab, 16)
    status, logits, _ = model.step(prompt)
    assert status == 0
    sample = logits[-1][::1000].copy()
    ids, top_ids, top_logits = [], [], []
    row = logits[-1]
    for _ in range(32):
        token = O.argmax(row)
        ids.append(token)
        i, v = top(row, 8)
        top_ids.append(i)
        top_logits.append(v)
        status, logits, _ = model.step(np.array([token], np.int32))
        assert status == 0
        row = logits[0]
    model.close()
    return {"prompt": prompt, "ids": np.array(ids, np.int32), "top_ids": np.stack(top_ids),
            "top_logits": np.stack(top_logits), "prompt_row_every_1000th": sample}


VARIED_SEED = 0x6A00
WHICH = (O.DBG_NORMALISED, O.DBG_ATTENDED, O.DBG_ACTIVATED)


def varied_sigma(model, index):
    """Spreads under which the greedy ids of the Gemma-2B shape change from
    step to step: embedding 0.02, norms 0.1, projections 3 / sqrt(fan in)."""
    if index == 0:
        return 0.02
    if model.is_norm(index):
        return 0.1
    role = (index - 1) % O.PER_LAYER
    fan_in = {O.T_O: model.shape.heads * model.shape.head_dim,
              O.T_DOWN: model.shape.intermediate}.get(role, model.shape.width)
    return 3.0 / np.sqrt(fan_in)


def q8_digest(q, s) -> bytes:
    return hashlib.sha256(np.ascontiguousarray(q).view(np.uint8).tobytes()
                          + np.ascontiguousarray(s).astype("<u2").tobytes()).digest()


def q8_digests(model):
    """[layers + 1, 3, 32] SHA-256 digests of the last row's Q8 product inputs:
    per layer (normalised, attended, activated); the final norm's row last
    (the other two left zero)."""
    layers = model.shape.layers
    out = np.zeros((layers + 1, 3, 32), np.uint8)
    for layer in range(layers):
        for k, which in enumerate(WHICH):
            out[layer, k] = np.frombuffer(q8_digest(*model.debug_q(which, layer)), np.uint8)
    out[layers, 0] = np.frombuffer(q8_digest(*model.debug_q(O.DBG_NORMALISED, layers)), np.uint8)
    return out


def greedy(model, prompt, steps, digest_steps=()):
    """The greedy loop by hand (Gemma.cpp:459-543 without the EOS stop): the
    prompt step with its last row's logits, then a step a token; each step's
    top-8 ids and logits and top-2 margin, and the Q8 digests of the last
    prompt row (index 0 of `digests`) and of the steps in digest_steps."""
    if len(prompt) > 1:  # the blocked step: the single steps' bits, far faster
        assert model.step_block(prompt[:-1], 0)[0] == 0
    status, logits, _ = model.step(prompt[-1:])
    assert status == 0
    digests = [q8_digests(model)]
    row = logits[0]
    prompt_sample = row[::1000].copy()
    ids, top_ids, top_logits, margins = [], [], [], []
    for step in range(steps):
        token = O.argmax(row)
        ids.append(token)
        i, v = top(row, 8)
        top_ids.append(i)
        top_logits.append(v)
        margins.append(v[0] - v[1])
        if step + 1 == steps:
            break
        status, logits, _ = model.step(np.array([token], np.int32))
        assert status == 0
        row = logits[0]
        if step + 1 in digest_steps:
            digests.append(q8_digests(model))
    return {"prompt": np.asarray(prompt, np.int32), "ids": np.array(ids, np.int32),
            "top_ids": np.stack(top_ids), "top_logits": np.stack(top_logits),
            "margins": np.array(margins, np.float32), "prompt_row_every_1000th": prompt_sample,
            "digests": np.stack(digests), "digest_steps": np.array(digest_steps, np.int32)}


def synthetic_gemma(layers, max_positions):
    model = O.Model(O.gemma_2b_shape(layers=layers, max_positions=max_positions), O.MODE_Q8)
    assert model.fill_synthetic() == 0
    return model


def gemma_ctx512():
    model = synthetic_gemma(18, 1024)
    prompt = O.prompt_ids(0xC0FFEE + 2, model.shape.vocab, 512)
    return greedy(model, prompt, 256)


def gemma_prefill2048():
    """Rows 0, 1023 and 2047 of the 2048-token prompt, stepped so that the
    oracle's last-row intermediates are those rows'."""
    model = synthetic_gemma(18, 2048)
    prompt = O.prompt_ids(0xC0FFEE + 3, model.shape.vocab, 2048)
    digests = []
    assert model.step(prompt[:1], want_logits=False)[0] == 0
    digests.append(q8_digests(model))
    assert model.step_block(prompt[1:1024], 0)[0] == 0
    digests.append(q8_digests(model))
    assert model.step_block(prompt[1024:2047], 0)[0] == 0
    status, logits, _ = model.step(prompt[2047:])
    assert status == 0
    digests.append(q8_digests(model))
    row = logits[0]
    i, v = top(row, 64)
    return {"prompt": prompt, "rows": np.array([0, 1023, 2047], np.int32),
            "digests": np.stack(digests), "top_ids": i, "top_logits": v,
            "every_1000th": row[::1000].copy()}


def gemma_varied18():
    model = O.Model(O.gemma_2b_shape(layers=18, max_positions=256), O.MODE_Q8)
    for index in range(model.tensor_count):
        values = O.normal_fill(VARIED_SEED + index, varied_sigma(model, index),
                               model.tensor_elements(index))
        assert model.set_tensor(index, values) == 0
    prompt = O.prompt_ids(0xC0FFEE + 7, model.shape.vocab, 64)
    return greedy(model, prompt, 48, digest_steps=(24,))


def gemma_varied18_ctx560():
    model = O.Model(O.gemma_2b_shape(layers=18, max_positions=1024), O.MODE_Q8)
    for index in range(model.tensor_count):
        values = O.normal_fill(VARIED_SEED + index, varied_sigma(model, index),
                               model.tensor_elements(index))
        assert model.set_tensor(index, values) == 0
    prompt = O.prompt_ids(0xC0FFEE + 9, model.shape.vocab, 560)
    return greedy(model, prompt, 24, digest_steps=(1, 12, 23))


def gemma_long8192():
    model = synthetic_gemma(18, 8192)
    prompt = O.prompt_ids(0xC0FFEE + 4, model.shape.vocab, 8064)
    out = greedy(model, prompt, 128)
    assert model.position == 8191
    return out


FULL_SIZE = {"ctx512": gemma_ctx512, "prefill2048": gemma_prefill2048,
             "varied18": gemma_varied18, "varied18_ctx560": gemma_varied18_ctx560,
             "long8192": gemma_long8192}


def main():
    wanted = sys.argv[1:]
    if wanted:
        for name in wanted:
            np.savez_compressed(os.path.join(HERE, f"gemma_{name}.npz"), **FULL_SIZE[name]())
            print(f"wrote gemma_{name}.npz", flush=True)
        return
    values = int8_block_inputs()
    np.savez_compressed(os.path.join(HERE, "int8_blocks.npz"), values=values,
                        stored=O.quantize_int8_blocks(values))
    cos, sin = O.rotary_table(8192, 256)
    rows = np.array([0, 1, 8191])
    np.savez_compressed(os.path.join(HERE, "rotary.npz"), positions=rows, cos=cos[rows],
                        sin=sin[rows])
    np.savez_compressed(os.path.join(HERE, "small_model.npz"), prompt=np.array(PROMPT),
                        **small_model())
    np.savez_compressed(os.path.join(HERE, "two_layer_gemma.npz"), **two_layer_gemma())


if __name__ == "__main__":
    main()
