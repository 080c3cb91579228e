"""The oracle's restatement of the sampler (Sampler.cpp:78-213), pinned by the
reference's own cases (Tests/Sampling/SamplerTests.cpp): greedy and its ties,
the mask, each cut's degenerate setting, top-k and top-p membership,
frequencies against a softmax spelled out here, temperature, seeds, and the
vocabulary-width row.  The draws are Sampler::uniform over std::mt19937_64,
whose outputs the oracle's format tests pin to the standard's known answers."""
import numpy as np

import oracle as O


def logits_for(probabilities):
    return np.log(np.array(probabilities, dtype=np.float64)).astype(np.float32)


def reference_softmax(logits, temperature):
    scaled = logits.astype(np.float64) / temperature
    w = np.exp(scaled - scaled.max())
    return w / w.sum()


def counts(sampler, logits, draws, mask=None):
    out = np.zeros(len(logits), dtype=np.int64)
    for _ in range(draws):
        out[sampler.sample(logits, mask)] += 1
    return out


def test_greedy_and_ties():
    assert O.Sampler().sample(np.array([0.1, 2.5, -1.0, 2.4], np.float32)) == 1
    assert O.Sampler().sample(np.array([1, 3, 3, 2, 3], np.float32)) == 1


def test_mask():
    logits = np.array([0, 5, 4, 1], np.float32)
    assert O.argmax(logits, np.array([0, 1, 0, 0], np.float32)) == 2
    assert O.argmax(logits, np.array([0, 1, 1, 0], np.float32)) == 3
    s = O.Sampler(temperature=2.0, seed=5)
    got = counts(s, logits, 10000, np.array([0, 1, 1, 0], np.float32))
    assert got[1] == 0 and got[2] == 0
    everything = np.ones(4, np.float32)
    assert O.Sampler(temperature=1.0, seed=11).sample(logits, everything) == 0
    assert O.Sampler().sample(logits, everything) == 0


def test_each_cut_reduces_to_greedy():
    logits = np.array([0.5, 3.0, 2.0, 2.99, -4.0], np.float32)
    for seed in range(8):
        for s in (O.Sampler(0.0, seed=seed), O.Sampler(1.0, top_k=1, seed=seed),
                  O.Sampler(1.0, top_p=1e-6, seed=seed)):
            assert all(s.sample(logits) == 1 for _ in range(100))


def test_top_k():
    logits = np.array([1, 4, 2, 3.5, 0, 3.9, -2, 2.2], np.float32)
    got = counts(O.Sampler(1.0, top_k=3, seed=7), logits, 10000)
    assert all(got[i] == 0 for i in (0, 2, 4, 6, 7))
    assert all(got[i] > 0 for i in (1, 3, 5))


def test_top_p_keeps_the_boundary_token():
    logits = logits_for([0.4, 0.3, 0.2, 0.1])
    draws = 20000
    got = counts(O.Sampler(1.0, top_p=0.5, seed=3), logits, draws)
    assert got[0] > 0 and got[1] > 0 and got[2] == 0 and got[3] == 0
    assert np.allclose(got / draws, [0.4 / 0.7, 0.3 / 0.7, 0, 0], atol=0.02)


def test_frequencies_and_temperature():
    draws = 20000
    logits = logits_for([0.5, 0.25, 0.15, 0.1])
    got = counts(O.Sampler(1.0, seed=12345), logits, draws)
    assert np.allclose(got / draws, reference_softmax(logits, 1.0), atol=0.02)
    logits = np.array([0, 1, 2, -1], np.float32)
    for t in (0.5, 1.0, 2.0):
        got = counts(O.Sampler(t, seed=808), logits, draws)
        assert np.allclose(got / draws, reference_softmax(logits, t), atol=0.02)


def test_seeds():
    logits = logits_for([0.5, 0.25, 0.15, 0.1])

    def sequence(**options):
        s = O.Sampler(**options)
        return [s.sample(logits) for _ in range(200)]

    first = sequence(temperature=1.0, seed=4242)
    assert first == sequence(temperature=1.0, seed=4242)
    assert first != sequence(temperature=1.0, seed=4243)
    assert sequence(temperature=1.0, top_k=3, seed=77) == sequence(temperature=1.0, top_k=3, seed=77)


def test_uniform_draws_are_the_top_53_bits():
    engine = (O.ctypes.c_uint64 * 313)()
    O.lib().gor_mt64_seed(engine, 4242)
    raw = [O.lib().gor_mt64_next(engine) for _ in range(5)]
    assert list(O.uniform_draws(4242, 5)) == [(r >> 11) * 2.0 ** -53 for r in raw]


def test_vocabulary_width_row():
    vocab, keep = 256000, 40
    logits = (np.sin(np.arange(vocab, dtype=np.float32) * np.float32(0.7)) * np.float32(6)).astype(np.float32)
    ranked = sorted(range(vocab), key=lambda t: (-float(logits[t]), t))[:keep]
    s = O.Sampler(0.8, top_k=keep, seed=99)
    assert all(s.sample(logits) in set(ranked) for _ in range(200))
