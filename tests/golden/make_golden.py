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
"""
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


def main():
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
