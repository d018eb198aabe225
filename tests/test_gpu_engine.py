"""The decode engine on the GPU, through the l3m.h API, against the reference and the oracle.

- Greedy tokens of the benchmark configurations (first 64 steps) must equal those of fpedd/l3m's scalar
  engine (tests/golden/decode.json, written by the reference built from source); the GPU fp32 reference
  path must reproduce the reference's --ref tokens.
- Logits after the prompt: argmax equal, KL(oracle || gpu) < 0.01 nats (the reference's `check` bar,
  main.c:291), and a max-abs bound relative to max|logit| (SPREAD below says why it is not 1e-3).
- The stop rules, callbacks, perf counters and run-to-run determinism of engine.c:322-362, 549-602.
"""
import hashlib
import os

import numpy as np
import pytest

import l3m_amd as A

pytestmark = pytest.mark.gpu
SMALL = A.Config("tiny", dim=128, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=256, vocab=512, ctx=64, dtype="q8_0")


def kl(lr, lf):
    lr, lf = np.float64(lr), np.float64(lf)
    pr = np.exp(lr - lr.max()); pr /= pr.sum()
    lpr = lr - lr.max() - np.log(np.exp(lr - lr.max()).sum())
    lpf = lf - lf.max() - np.log(np.exp(lf - lf.max()).sum())
    return float((pr * (lpr - lpf)).sum())


def golden_ids(golden):
    return [f"{c['config']}-{c['dtype']}" for c in golden["cases"]]


@pytest.fixture(scope="module")
def golden_cases(golden, models):
    out = []
    for c in golden["cases"]:
        path = models.get(c["config"], c["dtype"], seed=golden["seed"])
        assert hashlib.sha256(path.read_bytes()).hexdigest() == c["sha256"], "generator bytes changed"
        out.append((c, path))
    return out


# Post-prompt logits of the quantized configs legitimately spread at the level of the int8 activation
# quantization: fpedd/l3m's own avx2/avx512 tables differ from its scalar table by up to 1.03% of max|logit|
# on these models (stories42M q8_0), because any rounding difference flips a few rint() decisions of
# the per-block activation quantization and the flips cascade through the layers. bf16 and f32 paths,
# which do not quantize activations, agree to ~1e-6. So the engine bar is the reference's own `check`
# rule (same argmax, KL < 0.01 nats, main.c:291) plus a max-abs bound of 2% of max|logit|.
SPREAD = {"bf16": 1e-3, "f32": 1e-4, "q8_0": 0.02, "q4_0": 0.02, "mxfp4": 0.02}
# A greedy step whose top-2 margin in the reference is under 0.5% of max|logit| is a near-tie: the
# reference's own avx512 table leaves its scalar table exactly there on stories110M q4_0 (step 33).
NEAR_TIE = 0.005


@pytest.mark.parametrize("i", range(5))
def test_greedy_tokens_match_reference(golden_cases, oracle, i):
    c, path = golden_cases[i]
    print(f"case {c['config']} {c['dtype']}", flush=True)
    m = A.Model(path)
    toks = m.generate(c["prompt"], len(c["scalar_tokens"]))
    # Identical through the first near-tie: a step whose top-2 margin in the reference is inside the
    # activation-quantization spread may legitimately go either way (the reference's own SIMD table
    # leaves its scalar table at such steps, recorded as simd_agree).
    ties = [i for i, mg in enumerate(c["scalar_margins"]) if mg < NEAR_TIE]
    must = ties[0] if ties else len(toks)
    agree = next((i for i, (a, b) in enumerate(zip(toks, c["scalar_tokens"])) if a != b), len(toks))
    print(f"greedy agreement {agree} of {len(toks)} (first near-tie at {must}, reference SIMD agrees {c['simd_agree']})", flush=True)
    assert agree >= must
    m.generate(c["prompt"], 0)
    lg = m.logits
    om = oracle.load(path)
    om.generate(c["prompt"], 0)
    lo = om.logits()
    # the oracle reproduces the reference's scalar engine bit for bit on this box too
    assert hashlib.sha256(lo.tobytes()).hexdigest() == c["scalar_prompt_logits"]["sha256"]
    assert int(np.argmax(lg)) == c["scalar_prompt_logits"]["argmax"]
    assert kl(lo, lg) < 0.01
    err = float(np.abs(lg - lo).max() / np.abs(lo).max())
    print(f"logits max-abs / max|logit| = {err:.2e}, KL = {kl(lo, lg):.2e}", flush=True)
    assert err <= SPREAD[c["dtype"]]
    m.close()


@pytest.mark.parametrize("i", [0, 2])
def test_reference_mode_matches_reference_ref_path(golden_cases, i):
    c, path = golden_cases[i]
    m = A.Model(path, reference=True)
    assert "reference fp32" in m.describe()
    toks = m.generate(c["prompt"], 32)
    assert toks == c["ref_tokens"][:32]
    m.close()


def test_fast_vs_reference_mode_check(models):
    """l3m check semantics: quantized GPU path vs the fp32 GPU path after the prompt."""
    path = models.get("stories110M", "q4_0")
    ids = A.prompt(1, 32000, 4)
    fast, ref = A.Model(path), A.Model(path, reference=True)
    fast.generate(ids, 0)
    ref.generate(ids, 0)
    lf, lr = fast.logits, ref.logits
    assert int(np.argmax(lf)) == int(np.argmax(lr)) and kl(lr, lf) < 0.01


@pytest.mark.parametrize("dtype", ["f32", "bf16", "q8_0", "q4_0", "mxfp4"])
def test_small_model_every_position_matches_oracle(oracle, models, dtype):
    """A lively tiny GQA model (larger weights, jittered norms): tokens and logits at every step vs the oracle."""
    path = models.get(SMALL, dtype, seed=3, std=0.08, norm_jitter=0.2)
    ids = A.prompt(3, SMALL.vocab, 5)
    gpu, om = A.Model(path), oracle.load(path)
    want = om.generate(ids, 40)
    got = gpu.generate(ids, 40)
    assert got == want
    lo, lg = om.logits(), gpu.logits
    assert int(np.argmax(lg)) == int(np.argmax(lo)) and kl(lo, lg) < 0.01
    assert np.abs(lg - lo).max() <= SPREAD[dtype] * np.abs(lo).max()
    # the reference path too
    gref, oref = A.Model(path, reference=True), oracle.load(path, ref=True)
    assert gref.generate(ids, 40) == oref.generate(ids, 40)
    assert np.abs(gref.logits - oref.logits()).max() <= 1e-4 * np.abs(oref.logits()).max()


def test_runs_are_bitwise_identical_and_graph_matches_eager(models):
    path = models.get(SMALL, "q4_0", seed=4, std=0.08, norm_jitter=0.2)
    ids = A.prompt(4, SMALL.vocab, 3)
    m = A.Model(path)
    a = m.generate(ids, 30); la = m.logits
    b = m.generate(ids, 30); lb = m.logits
    assert a == b and np.array_equal(la, lb)
    os.environ["L3M_GRAPH"] = "0"
    try:
        e = A.Model(path)
    finally:
        del os.environ["L3M_GRAPH"]
    assert e.generate(ids, 30) == a and np.array_equal(e.logits, la)


def test_ctx_limits_generation(models):
    path = models.get(SMALL, "q8_0", seed=5)
    m = A.Model(path, ctx=16)
    assert m.ctx == 16
    assert len(m.generate([1], 100)) == 16 - 1
    assert len(m.generate([1, 2, 3], 100)) == 16 - 3
    with pytest.raises(ValueError):
        m.generate(list(range(16)), 10)


def test_callback_stop_logits_and_perf(oracle, models):
    path = models.get(SMALL, "q8_0", seed=6, std=0.08, norm_jitter=0.2)
    ids = A.prompt(6, SMALL.vocab, 4)
    m = A.Model(path)
    m.perf()                                   # start the counters from here
    stop_after, heard = 5, []

    def listener(tok):
        heard.append(tok)
        return len(heard) < stop_after

    out = m.generate(ids, 50, on_token=listener)
    assert out == heard
    assert len(out) == stop_after
    counters = m.perf()
    assert counters["tokens"] == len(ids) - 1 + stop_after     # forward passes, the prompt included
    assert counters["ns_token"] > 0 < counters["bytes_token"]
    assert np.isnan(list(m.perf().values())).all()             # nothing ran since the last read
    # logits are the prediction after the last token fed: position len(ids) + 3
    om = oracle.load(path)
    full = om.generate(ids, 4)
    assert full == out[:4]
    assert int(np.argmax(m.logits)) == out[4] and kl(om.logits(), m.logits) < 0.01
    assert np.abs(m.logits - om.logits()).max() <= SPREAD["q8_0"] * np.abs(om.logits()).max()


def test_bad_prompt_ids(models):
    m = A.Model(models.get(SMALL, "q8_0", seed=5))
    with pytest.raises(ValueError):
        m.generate([SMALL.vocab], 2)
    assert m.generate([], 2) == []


@pytest.mark.parametrize("key", [("tiny", "q4_0"), ("stories15M", "bf16"), ("stories110M", "q4_0"), ("smollm2", "mxfp4")],
                         ids=lambda k: f"{k[0]}-{k[1]}")
def test_persistent_kernel_equals_graph_path(models, monkeypatch, key):
    """The persistent decode kernel runs the same blocks in the same order as the one-graph-per-step path:
    tokens and final logits are bit-identical, over a launch boundary (more than 64 steps) and the
    restart of a second generate."""
    cfg = SMALL if key[0] == "tiny" else A.CONFIGS[key[0]]
    path = models.get(cfg, key[1], seed=3)
    ids = A.prompt(3, cfg.vocab, cfg.n_prompt)
    n = min(cfg.ctx - len(ids) - 1, 70)
    out = {}
    for persist in ("1", "0"):
        monkeypatch.setenv("L3M_PERSIST", persist)
        with A.Model(path) as m:
            if persist == "1":
                assert m.persistent, "the persistent kernel should fit this model"
            else:
                assert not m.persistent
            first = m.generate(ids, n)
            second = m.generate(ids[:2], 5)
            out[persist] = (first, second, m.logits)
    assert out["1"][0] == out["0"][0] and out["1"][1] == out["0"][1]
    np.testing.assert_array_equal(out["1"][2], out["0"][2])
