"""Batched prompt prefill on the GPU (int8 GEMMs on the matrix cores), through the l3m.h API.

A prompt of at least L3M_PREFILL_MIN (8) tokens runs its positions before the last in one batched pass
that fills the K/V cache; decoding then starts at the last prompt token. The logits after the prompt
must meet the engine bar of test_gpu_engine.py against the oracle (the reference's token-by-token order)
and against the GPU's own token-by-token path (L3M_PREFILL=0): equal argmax, KL < 0.01 nats, max-abs
within 2% of max|logit| (the int8 activation noise floor of the quantized paths). Prompts of 8 (the
threshold: 7 positions, less than one 16-token group of the GEMM), 9 and 17 (a group boundary), 40 and 100
tokens cover one to seven 16-token groups of the GEMM, and 65 ends exactly at the attention's second
64-position chunk; head dims of 32 and 64 prepare the attention output inside the attention kernel, hd 48 in one of
its own. q4_0 and
mxfp4 bodies run the same int8 GEMM on q8_0 copies of their matrices with the same values (an mxfp4 block's
scale 2^(e-128) is an f16 and its doubled e2m1 codes are int8).
"""
import numpy as np
import pytest

import l3m_amd as A

pytestmark = pytest.mark.gpu
GQA = A.Config("pf_gqa", dim=192, n_layers=3, n_heads=6, n_kv_heads=2, ffn_dim=512, vocab=512, ctx=128, dtype="q8_0")
MHA = A.Config("pf_mha", dim=256, n_layers=2, n_heads=4, n_kv_heads=4, ffn_dim=640, vocab=512, ctx=128, dtype="q4_0")
MX = A.Config("pf_mx", dim=192, n_layers=2, n_heads=6, n_kv_heads=3, ffn_dim=512, vocab=512, ctx=128, dtype="mxfp4")
# hd 48: the attention output's blocks span heads, so it is prepared by a kernel of its own
HD48 = A.Config("pf_hd48", dim=192, n_layers=3, n_heads=4, n_kv_heads=2, ffn_dim=512, vocab=512, ctx=128, dtype="q8_0")


def kl(lr, lf):
    lr, lf = np.float64(lr), np.float64(lf)
    pr = np.exp(lr - lr.max()); pr /= pr.sum()
    lpr = lr - lr.max() - np.log(np.exp(lr - lr.max()).sum())
    lpf = lf - lf.max() - np.log(np.exp(lf - lf.max()).sum())
    return float((pr * (lpr - lpf)).sum())


def bf16(u):
    return (np.asarray(u, np.uint32) << 16).view(np.float32).astype(np.float64)


def ulps(a, b):
    """Distance in bf16 units in the last place (values of one sign; a sign change counts through zero)."""
    def key(u):
        u = np.asarray(u, np.int64)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(key(a) - key(b))


def close(a, b):
    return int(np.argmax(a)) == int(np.argmax(b)) and kl(b, a) < 0.01 and np.abs(a - b).max() <= 0.02 * np.abs(b).max()


@pytest.mark.parametrize("n_prompt", [8, 9, 17, 40, 65, 100])
@pytest.mark.parametrize("cfg", [GQA, MHA, MX, HD48], ids=["q8_0-gqa", "q4_0-mha", "mxfp4-gqa", "q8_0-hd48"])
def test_prefill_logits(models, oracle, monkeypatch, cfg, n_prompt):
    print(f"case {cfg.name} prompt {n_prompt}", flush=True)
    path = models.get(cfg, cfg.dtype, seed=9, std=0.05, norm_jitter=0.1)
    ids = A.prompt(9, cfg.vocab, n_prompt)
    fast = A.Model(path)
    fast.generate(ids, 0)
    assert fast.prefilled == n_prompt - 1
    lf = fast.logits
    monkeypatch.setenv("L3M_PREFILL", "0")
    step = A.Model(path)
    step.generate(ids, 0)
    assert step.prefilled == 0
    ls = step.logits
    om = oracle.load(path)
    om.generate(ids, 0)
    lo = om.logits()
    assert close(lf, lo), (kl(lo, lf), np.abs(lf - lo).max() / np.abs(lo).max())
    assert close(lf, ls)
    # the K/V rows the prefill wrote, against the oracle's (the reference's token-by-token order) and the
    # GPU's own token-by-token rows
    hd, P = cfg.dim // cfg.n_heads, n_prompt - 1
    worst = {}
    for layer in range(cfg.n_layers):
        for kvh in range(cfg.n_kv_heads):
            kp, vp = fast.kv_rows(layer, kvh, 0, P, hd)
            ks, vs = step.kv_rows(layer, kvh, 0, P, hd)
            ko, vo = om.kv_rows(layer, kvh, 0, P, hd)
            for name, got_, tok_, ora in (("k", kp, ks, ko), ("v", vp, vs, vo)):
                g, t, o = bf16(got_), bf16(tok_), bf16(ora)
                scale = np.abs(o).max()
                assert np.abs(g - o).max() <= 0.02 * scale, (layer, kvh, name)
                assert np.abs(g - t).max() <= 0.02 * scale, (layer, kvh, name)
                if layer == 0:                        # before activation rounding can cascade: nearly exact
                    assert np.abs(g - o).max() <= 0.005 * scale, (layer, kvh, name)
                    assert np.mean(ulps(got_, ora) <= 1) >= 0.99, (layer, kvh, name)
                worst[name] = max(worst.get(name, 0.0), float(np.abs(g - o).max() / scale))
    print(f"prefill K/V vs oracle, worst max-abs / max|x|: {worst}", flush=True)
    # the continuation decodes over the prefilled cache: at every one of its 8 steps the GPU's token is the
    # oracle's argmax given the same prefix (its top two at a near-tie)
    got = fast.generate(ids, 8)
    assert fast.prefilled == P
    om2 = oracle.load(path)
    seq = list(ids) + got
    for k in range(len(got)):
        pos = len(ids) - 1 + k
        if k == 0:
            for p in range(pos):
                om2.forward(seq[p], p, logits=False)
        lg = om2.forward(seq[pos], pos).astype(np.float64)
        order = np.argsort(-lg, kind="stable")
        lv = np.sort(lg)
        tie = (lv[-1] - lv[-2]) / np.abs(lv).max() < 0.005
        assert got[k] == order[0] or (tie and got[k] == order[1]), (k, got, order[:2])


def test_prefill_graph_replays_equal_loose_launches(models, monkeypatch):
    """The prefill runs as one captured graph per prompt length (L3M_PREFILL_GRAPH=0: the same launches
    one by one). Every call, including replays of a length captured earlier with decoding and other lengths
    run in between, gives logits and K/V rows bit-identical to the loose launches of the same prompt."""
    cfg = GQA
    path = models.get(cfg, cfg.dtype, seed=9, std=0.05, norm_jitter=0.1)
    hd = cfg.dim // cfg.n_heads
    graph = A.Model(path)
    monkeypatch.setenv("L3M_PREFILL_GRAPH", "0")
    loose = A.Model(path)
    for i, n_prompt in enumerate([40, 100, 40, 57, 100, 40]):
        print(f"call {i}: prompt {n_prompt}", flush=True)
        ids = A.prompt(20 + i, cfg.vocab, n_prompt)
        got = graph.generate(ids, 3)
        want = loose.generate(ids, 3)
        assert graph.prefilled == loose.prefilled == n_prompt - 1
        assert got == want
        assert np.array_equal(graph.logits, loose.logits)
        for layer in range(cfg.n_layers):
            for kvh in range(cfg.n_kv_heads):
                kg, vg = graph.kv_rows(layer, kvh, 0, n_prompt - 1, hd)
                kl_, vl = loose.kv_rows(layer, kvh, 0, n_prompt - 1, hd)
                assert np.array_equal(kg, kl_) and np.array_equal(vg, vl), (i, layer, kvh)


LONG = A.Config("pf_long", dim=128, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=256, vocab=512, ctx=256, dtype="q8_0")


def test_prefill_past_128_positions(models, oracle, monkeypatch):
    """A 200-token prompt at ctx 256: 199 prefilled positions, past the 128-slot logits ring and over four of
    the attention's 64-position chunks. The logits after the prompt meet the engine bar against the oracle
    and the GPU's token-by-token path, and each of the 30 greedy tokens that follow is the oracle's argmax
    given the same prefix (its second at a near-tie)."""
    path = models.get(LONG, "q8_0", seed=3, std=0.08, norm_jitter=0.2)
    ids = A.prompt(7, LONG.vocab, 200)
    om = oracle.load(path, ctx=256)
    om.generate(ids, 0)
    lo = om.logits()
    with A.Model(path, ctx=256) as m:
        m.generate(ids, 0)
        assert m.prefilled == 199
        lf = m.logits
        got = m.generate(ids, 30)
    om2, seq = oracle.load(path, ctx=256), list(ids) + got
    for p in range(len(ids) - 1):
        om2.forward(seq[p], p, logits=False)
    for k in range(len(got)):
        pos = len(ids) - 1 + k
        lg = om2.forward(seq[pos], pos).astype(np.float64)
        order, lv = np.argsort(-lg, kind="stable"), np.sort(lg)
        tie = (lv[-1] - lv[-2]) / np.abs(lv).max() < 0.005
        assert got[k] == order[0] or (tie and got[k] == order[1]), (k, got[k], order[:2])
    monkeypatch.setenv("L3M_PREFILL", "0")
    with A.Model(path, ctx=256) as m:
        m.generate(ids, 0)
        assert m.prefilled == 0
        ls = m.logits
    assert close(lf, lo), (kl(lo, lf), np.abs(lf - lo).max() / np.abs(lo).max())
    assert close(lf, ls)


def test_prefill_graph_cache_replaces_the_oldest(models, monkeypatch):
    """More prompt lengths than the eight captured graphs a model keeps: eleven lengths in turn, then the
    first three again (each replaced since and captured anew) and the last (still kept). Every call's tokens
    and logits equal the loose launches' bit for bit."""
    path = models.get(GQA, GQA.dtype, seed=9, std=0.05, norm_jitter=0.1)
    graph = A.Model(path)
    monkeypatch.setenv("L3M_PREFILL_GRAPH", "0")
    loose = A.Model(path)
    lengths = list(range(10, 32, 2))
    for i, n_prompt in enumerate(lengths + lengths[:3] + lengths[-1:]):
        ids = A.prompt(40 + n_prompt, GQA.vocab, n_prompt)
        got, want = graph.generate(ids, 2), loose.generate(ids, 2)
        assert graph.prefilled == loose.prefilled == n_prompt - 1
        assert got == want, (i, n_prompt)
        assert np.array_equal(graph.logits, loose.logits), (i, n_prompt)
    graph.close(); loose.close()
