"""Temperature sampling on the GPU (engine.c:98-101, 284-319, 555), through the l3m.h API.

- Every sampled token equals the oracle's pick (the reference path's order, pinned against fpedd/l3m in
  test_cpu_sampling.py) from the logits the GPU computed at that position, with the generator advanced
  once per token from the generate call's seed: on the persistent kernel and on the one-graph-per-step
  path, for quantized and bf16 models. (The GPU's expf is not glibc's: a pick could differ only where
  u * z falls within a few float ulps of a boundary of the running sum.)
- The first sampled token over many seeds follows softmax(logits / T) (chi-square, as the reference's
  test_sampling_distribution).
- Greedy decoding is unchanged by a sampled call before it, and the same seed gives the same tokens.
"""
import numpy as np
import pytest

import l3m_amd as A

pytestmark = pytest.mark.gpu
CFG = A.Config("samp", dim=128, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=256, vocab=512, ctx=128, dtype="q4_0")


def check_against_oracle(m, oracle, ids, temp, seed, n):
    toks = m.generate(ids, n, temperature=temp, seed=seed)
    st = oracle.seed_state(seed)
    for k, tok in enumerate(toks):
        want, st = oracle.sample(m.logits_at(len(ids) - 1 + k), temp, st)
        assert tok == want, f"seed {seed}, token {k}"
    if len(toks) < n:                                 # stopped: the next pick was EOS or BOS
        want, st = oracle.sample(m.logits_at(len(ids) - 1 + len(toks)), temp, st)
        assert want in (m.eos, m.bos)
    return toks


@pytest.mark.parametrize("persist", ["1", "0"])
@pytest.mark.parametrize("dtype", ["q4_0", "q8_0", "bf16"])
def test_sampled_tokens_match_oracle(models, oracle, monkeypatch, dtype, persist):
    print(f"case {dtype} persist={persist}", flush=True)
    monkeypatch.setenv("L3M_PERSIST", persist)
    path = models.get(CFG, dtype, seed=6, std=0.05)
    m = A.Model(path)
    assert m.persistent == (persist == "1")
    ids = A.prompt(6, CFG.vocab, 5)
    seen = set()
    for temp in (1.0, 0.6):
        for seed in range(4):
            seen.add(tuple(check_against_oracle(m, oracle, ids, temp, seed, 48)))
    assert len(seen) > 4


@pytest.mark.parametrize("persist", ["1", "0"])
@pytest.mark.parametrize("arch,vocab", [("llama", 1001), ("gpt2", 50257)])
def test_sampled_any_vocabulary(models, oracle, monkeypatch, arch, vocab, persist):
    """Temperature sampling with a vocabulary that is not a multiple of 4 (GPT-2's 50257 among them): the
    GPU's picks equal the oracle's from the GPU's own logits, on the persistent kernel and on the
    one-graph-per-step path."""
    monkeypatch.setenv("L3M_PERSIST", persist)
    cfg = A.Config(f"samp{vocab}", dim=128, n_layers=2, n_heads=4, n_kv_heads=4 if arch == "gpt2" else 2, ffn_dim=256, vocab=vocab,
                   ctx=64, dtype="q8_0")
    path = models.get(cfg, "q8_0", seed=9, std=0.08, arch=arch)
    m = A.Model(path)
    assert m.persistent == (persist == "1")
    ids = A.prompt(9, vocab, 4)
    for seed in range(3):
        check_against_oracle(m, oracle, ids, 0.8, seed, 24)
    m.close()


def test_sampling_distribution(models):
    path = models.get(CFG, "q8_0", seed=8, std=0.2)
    m = A.Model(path)
    ids, temp, n = [3, 9], 0.8, 3000
    m.generate(ids, 0)
    lg = m.logits.astype(np.float64)
    p = np.exp((lg - lg.max()) / temp)
    p /= p.sum()
    p[m.eos] += p[m.bos]                              # both end generation
    p[m.bos] = 0
    counts = np.zeros(m.vocab)
    for seed in range(n):
        out = m.generate(ids, 1, temperature=temp, seed=seed)
        counts[out[0] if out else m.eos] += 1
    big = p * n >= 5
    obs = np.append(counts[big], counts[~big].sum())
    exp = np.append(p[big], p[~big].sum()) * n
    df = len(obs) - 1
    assert ((obs - exp) ** 2 / exp).sum() < df + 5 * np.sqrt(2 * df)


def test_seed_repeats_and_greedy_is_unchanged(models):
    path = models.get(CFG, "q4_0", seed=6, std=0.05)
    m = A.Model(path)
    ids = A.prompt(7, CFG.vocab, 4)
    greedy = m.generate(ids, 40)
    a = m.generate(ids, 40, temperature=0.9, seed=5)
    assert m.generate(ids, 40, temperature=0.9, seed=5) == a
    assert m.generate(ids, 40) == greedy              # the sampled calls leave no state behind


@pytest.mark.parametrize("persist", ["1", "0"])
def test_extreme_temperatures(models, oracle, monkeypatch, persist):
    """Temperatures far from 1 follow the reference's rules too: 1e-30 leaves weight only on the maximum
    (every other exponent is below -16), 1e-3 nearly so, 1e3 and 1e30 spread the weight over the whole
    vocabulary, and infinity makes every weight 1. The picks equal the oracle's from the GPU's logits."""
    monkeypatch.setenv("L3M_PERSIST", persist)
    path = models.get(CFG, "q8_0", seed=6, std=0.05)
    m = A.Model(path)
    ids = A.prompt(6, CFG.vocab, 5)
    greedy = m.generate(ids, 24)
    for temp in (1e-30, 1e-3, 1e3, 1e30, float("inf")):
        print(f"case temperature {temp} persist={persist}", flush=True)
        toks = check_against_oracle(m, oracle, ids, temp, 11, 24)
        if temp == 1e-30:
            assert toks == greedy
        if temp >= 1e3:
            assert len(set(toks)) > 12                  # spread over the vocabulary
    m.close()


def test_sampled_streamed_after_a_prefilled_prompt(models, oracle):
    """The three features together: a 40-token prompt through the batched prefill, temperature sampling on
    the device, and tokens handed to on_token as they come, with a stop after 20. Every pick equals the
    oracle's from the GPU's logits, and the stopped call's tokens are the first 20 of the same call without a
    callback."""
    path = models.get(CFG, "q8_0", seed=6, std=0.05)
    m = A.Model(path)
    ids = A.prompt(8, CFG.vocab, 40)
    full = check_against_oracle(m, oracle, ids, 0.9, 3, 60)
    assert m.prefilled == len(ids) - 1
    seen = []
    got = m.generate(ids, 60, temperature=0.9, seed=3, on_token=lambda t: seen.append(t) or len(seen) < 20)
    assert m.prefilled == len(ids) - 1
    assert got == seen == full[:20]
    st = oracle.seed_state(3)
    for k, tok in enumerate(got):
        want, st = oracle.sample(m.logits_at(len(ids) - 1 + k), 0.9, st)
        assert tok == want
    m.close()
