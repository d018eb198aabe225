"""Temperature sampling in the oracle (engine.c:98-101, 284-287, 364-379, 555), pinned without the GPU.

- Against fpedd/l3m built from source (oracle/_ref): generating with a temperature, the oracle's tokens
  equal the reference's on its --ref path (the same single-thread order) and on its multi-rank path, for
  8 seeds, as the reference's own test_sampling_matches_reference asserts of its two paths.
- Against the mathematics: the first draw of a seed from 64-bit integer arithmetic, the distribution of
  the picked token (a chi-square test against softmax(logits / T), as test_sampling_distribution does),
  and the special cases: temperature <= 0 or NaN is the first maximum, an overwhelming logit always wins.
"""
import numpy as np
import pytest

import l3m_amd as A

TINY = A.Config("samp", dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=128, vocab=256, ctx=64, dtype="f32")
MASK = (1 << 64) - 1


def xorshift64star(state):
    """One step of Vigna's xorshift64* in Python integers: (next state, 53-bit draw in [0, 1))."""
    state ^= state >> 12
    state ^= (state << 25) & MASK
    state ^= state >> 27
    return state, ((state * 0x2545F4914F6CDD1D) & MASK) >> 11


@pytest.mark.parametrize("seed", [0, 1, 7, 2**63 + 5, MASK])
def test_draws_follow_the_generator(oracle, seed):
    state = (seed * 0x9E3779B97F4A7C15 + 1) & MASK
    assert oracle.seed_state(seed) == state
    st = oracle.seed_state(seed)
    for _ in range(5):
        state, top = xorshift64star(state)
        u, st = oracle.rand01(st)
        assert st == state and u == top / 2.0**53 and 0.0 <= u < 1.0


def test_non_positive_temperature_is_the_first_maximum(oracle):
    x = np.array([0.5, 2.0, -1.0, 2.0, 1.5], np.float32)
    for t in (0.0, -1.0, float("nan")):
        tok, st = oracle.sample(x, t, 12345)
        assert tok == 1 and st == 12345                # no draw either


def test_an_overwhelming_logit_always_wins(oracle):
    x = np.zeros(64, np.float32)
    x[17] = 40.0                                      # every other weight is below e^-16 at T = 1
    st = oracle.seed_state(3)
    for _ in range(200):
        tok, st = oracle.sample(x, 1.0, st)
        assert tok == 17


@pytest.mark.parametrize("temp", [0.5, 1.0])
def test_sample_distribution(oracle, temp):
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1.5, 40).astype(np.float32)
    p = np.exp((x.astype(np.float64) - x.max()) / temp)
    p /= p.sum()
    n, st = 6000, oracle.seed_state(99)
    counts = np.zeros(len(x))
    for _ in range(n):
        tok, st = oracle.sample(x, temp, st)
        counts[tok] += 1
    big = p * n >= 5
    obs = np.append(counts[big], counts[~big].sum())
    exp = np.append(p[big], p[~big].sum()) * n
    df = len(obs) - 1
    assert ((obs - exp) ** 2 / exp).sum() < df + 5 * np.sqrt(2 * df)


@pytest.mark.parametrize("temp", [1.0, 0.7, 1e-30, 1e-3, 1e3, 1e30, float("inf")])
def test_sampled_generation_matches_reference(models, oracle, reference, temp):
    """The oracle's sampled generation equals the reference's, at ordinary temperatures and at the extremes
    (1e-30 keeps only the maximum, infinity makes every weight 1)."""
    path = models.get(TINY, "f32", seed=5, std=0.08)   # f32: both reference paths compute the same logits
    ids = A.prompt(5, TINY.vocab, 4)
    ref_path, ref_fast = reference.load(path, reference=True), reference.load(path, cpus=[0, 1, 2])
    om = oracle.load(path, ref=True)
    seen = set()
    for seed in range(8):
        want = ref_path.generate(ids, 32, temperature=temp, seed=seed)
        assert om.generate(ids, 32, temperature=temp, seed=seed) == want
        assert ref_fast.generate(ids, 32, temperature=temp, seed=seed) == want
        seen.add(tuple(want))
    if temp > 0.01:
        assert len(seen) > 1                          # the seed matters
    elif temp < 1e-20:
        assert len(seen) == 1                         # all weight on the maximum: the greedy tokens


@pytest.mark.parametrize("dtype", ["f32", "bf16", "q8_0", "q4_0"])
def test_gpt2_variant_matches_reference(models, oracle, reference, dtype):
    """The oracle's GPT-2 variant (LayerNorm with biases, learned positions, matrix biases, GELU MLP;
    engine.c:236-275, ops.c:20-27, 53-56) against fpedd/l3m built from source: its reference path bit for
    bit, its fast path to its own float rounding."""
    cfg = A.Config("g2", dim=64, n_layers=2, n_heads=4, n_kv_heads=4, ffn_dim=256, vocab=256, ctx=64, dtype=dtype)
    path = models.get(cfg, dtype, seed=3, std=0.08, arch="gpt2")
    ids = A.prompt(3, cfg.vocab, 5)
    r, o = reference.load(path, reference=True), oracle.load(path, ref=True)
    assert r.generate(ids, 12) == o.generate(ids, 12)
    assert np.array_equal(r.logits(), o.logits())
    rf, of = reference.load(path, cpus=[0]), oracle.load(path)
    assert rf.generate(ids, 12) == of.generate(ids, 12)
    lr, lo = rf.logits(), of.logits()
    assert np.abs(lr - lo).max() <= 1e-5 * np.abs(lr).max()
