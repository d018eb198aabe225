"""The GPT-2 variant on the GPU (LayerNorm with biases, learned positions, biases on every matrix, GELU
MLP without gate; model.h:19-26, engine.c:236-275), through the l3m.h API, against the oracle (pinned
bit-exact against the reference's --ref path in test_cpu_sampling.py). It runs on the persistent decode
kernel, whose tokens and logits equal the one-graph-per-step path's (L3M_PERSIST=0) bit for bit; the bar
against the oracle is the engine's: equal argmax, KL < 0.01 nats, max-abs within SPREAD of max|logit|
after the prompt, and the greedy tokens of the oracle until its first near-tie.
"""
import numpy as np
import pytest

import l3m_amd as A

pytestmark = pytest.mark.gpu
CFG = A.Config("g2gpu", dim=128, n_layers=2, n_heads=4, n_kv_heads=4, ffn_dim=512, vocab=512, ctx=64, dtype="q8_0")
SPREAD = {"f32": 1e-4, "bf16": 1e-3, "q8_0": 0.02, "q4_0": 0.02}


def kl(lr, lf):
    lr, lf = np.float64(lr), np.float64(lf)
    pr = np.exp(lr - lr.max()); pr /= pr.sum()
    lpr = lr - lr.max() - np.log(np.exp(lr - lr.max()).sum())
    lpf = lf - lf.max() - np.log(np.exp(lf - lf.max()).sum())
    return float((pr * (lpr - lpf)).sum())


def margin(logits):
    top = np.sort(logits)[-2:]
    return (top[1] - top[0]) / np.abs(logits).max()


@pytest.mark.parametrize("dtype", ["bf16", "q8_0", "q4_0", "f32"])
def test_gpt2_matches_oracle(models, oracle, dtype):
    print(f"case gpt2 {dtype}", flush=True)
    path = models.get(CFG, dtype, seed=5, std=0.06, norm_jitter=0.1, arch="gpt2")
    ids = A.prompt(5, CFG.vocab, 12)
    m, om = A.Model(path), oracle.load(path)
    assert m.persistent
    m.generate(ids, 0)
    assert m.prefilled == 0
    om.generate(ids, 0)
    lg, lo = m.logits, om.logits()
    assert int(np.argmax(lg)) == int(np.argmax(lo)) and kl(lo, lg) < 0.01
    assert np.abs(lg - lo).max() <= SPREAD[dtype] * np.abs(lo).max()
    got, want = m.generate(ids, 16), om.generate(ids, 16)
    # equal up to the first step whose top-2 margin in the oracle is a near-tie (0.5% of max|logit|)
    seq = list(ids)
    for k, (a, b) in enumerate(zip(got, want)):
        om.generate(seq, 0)
        if margin(om.logits()) < 0.005:
            break
        assert a == b, f"step {k}"
        seq.append(b)


def test_gpt2_reference_path(models, oracle):
    path = models.get(CFG, "q4_0", seed=5, std=0.06, norm_jitter=0.1, arch="gpt2")
    ids = A.prompt(6, CFG.vocab, 6)
    gref, oref = A.Model(path, reference=True), oracle.load(path, ref=True)
    assert gref.generate(ids, 16) == oref.generate(ids, 16)
    assert np.abs(gref.logits - oref.logits()).max() <= 1e-4 * np.abs(oref.logits()).max()


@pytest.mark.parametrize("dtype", ["q8_0", "bf16"])
def test_gptneo_without_qkv_biases(models, oracle, dtype):
    """GPT-Neo: an output bias but no q, k, v biases (the reference's test_attention_without_qkv_biases,
    test_engine.py:194-201). The oracle is teacher-forced along the GPU's greedy tokens: each is its argmax
    (its top two at a near-tie)."""
    print(f"case gptneo {dtype}", flush=True)
    path = models.get(CFG, dtype, seed=7, std=0.06, norm_jitter=0.1, arch="gptneo")
    ids = A.prompt(7, CFG.vocab, 9)
    m, om = A.Model(path), oracle.load(path)
    got = m.generate(ids, 20)
    seq = list(ids) + got
    for pos in range(len(seq) - 1):
        lg = om.forward(seq[pos], pos, logits=pos >= len(ids) - 1)
        if lg is None:
            continue
        k = pos - (len(ids) - 1)
        order = np.argsort(-lg.astype(np.float64), kind="stable")
        assert got[k] == order[0] or (margin(lg) < 0.005 and got[k] == order[1]), (k, got[k], order[:2])
        if k == 0:
            lo, lgpu = lg, m.logits_at(pos)
            assert kl(lo, lgpu) < 0.01 and np.abs(lgpu - lo).max() <= SPREAD[dtype] * np.abs(lo).max()


@pytest.mark.parametrize("arch,dtype", [("gpt2", "f32"), ("gpt2", "q4_0"), ("gptneo", "q8_0"), ("gptneo", "bf16")])
def test_persistent_kernel_equals_graph_path(models, monkeypatch, arch, dtype):
    """The GPT-2 family on the persistent kernel against the same model decoded one graph per step: the
    same greedy tokens and bit-identical logits at the end of each of three calls."""
    print(f"case {arch} {dtype}", flush=True)
    path = models.get(CFG, dtype, seed=11, std=0.06, norm_jitter=0.1, arch=arch)
    fast = A.Model(path)
    assert fast.persistent
    monkeypatch.setenv("L3M_PERSIST", "0")
    step = A.Model(path)
    assert not step.persistent
    for i, (n_prompt, n_new) in enumerate([(5, 40), (1, 62), (20, 10)]):
        ids = A.prompt(30 + i, CFG.vocab, n_prompt)
        assert fast.generate(ids, n_new) == step.generate(ids, n_new), i
        assert np.array_equal(fast.logits, step.logits), i


LONG = A.Config("g2long", dim=128, n_layers=2, n_heads=4, n_kv_heads=4, ffn_dim=512, vocab=512, ctx=300, dtype="q8_0")
TIE = {"f32": 1e-4, "bf16": 0.01, "q8_0": 0.02, "q4_0": 0.02}


@pytest.mark.parametrize("dtype", ["bf16", "q8_0"])
def test_gpt2_to_the_end_of_a_long_context(models, oracle, monkeypatch, dtype):
    """GPT-2 greedy decoding to the end of a 300-position context (three launches of the persistent kernel,
    learned position rows up to the last): teacher-forcing the oracle along the GPU's tokens, each is the
    oracle's argmax, or its second where the oracle's top-2 margin is inside the dtype's rounding spread;
    the one-graph-per-step path gives the same tokens and logits bit for bit."""
    path = models.get(LONG, dtype, seed=5, std=0.06, norm_jitter=0.1, arch="gpt2")
    ids = A.prompt(5, LONG.vocab, 5)
    out = {}
    for persist in ("1", "0"):
        monkeypatch.setenv("L3M_PERSIST", persist)
        with A.Model(path) as m:
            assert m.persistent == (persist == "1") and m.ctx == 300
            out[persist] = (m.generate(ids, 1000), m.logits)
    got = out["1"][0]
    assert len(got) == 300 - len(ids)
    om, seq, bad = oracle.load(path), list(ids) + got, []
    for pos in range(len(seq) - 1):
        lg = om.forward(seq[pos], pos, logits=pos >= len(ids) - 1)
        if lg is None:
            continue
        k = pos - (len(ids) - 1)
        order = np.argsort(-lg.astype(np.float64), kind="stable")
        if not (got[k] == order[0] or (margin(lg) < TIE[dtype] and got[k] == order[1])):
            bad.append(k)
    assert not bad, bad
    assert out["0"][0] == got
    np.testing.assert_array_equal(out["0"][1], out["1"][1])
