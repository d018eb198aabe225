"""CPU checks that pin the oracle (oracle/oracle.c, the checker of the GPU path) and the synthetic model
generator, without a GPU:

- the golden vectors of fpedd/l3m's own tests (tests/golden/ggml_blocks.json, from its
  tests/unit/test_export.py): ggml block bytes, bf16 round-to-nearest-even, the q8_0 rounding case;
- closed forms: the block definitions of src/model.h:58-60 and kernels.h:20-21 evaluated in float64,
  numpy's float16 conversion, textbook RMSNorm / RoPE / SiLU / softmax attention in float64;
- the reference built from its own sources (oracle/_ref, when present): activation prep, every gemv
  table entry and attend, and its scalar engine's greedy tokens and logits (tests/golden/decode.json,
  written by tests/golden/make_golden.py from that build).
"""
import hashlib
import json

import numpy as np
import pytest

import l3m_amd as A
from conftest import GOLDEN
from weights import BF16, F32, MXFP4, Q4_0, Q8_0, extremes, rows, to_bf16

BLOCKS = json.loads((GOLDEN / "ggml_blocks.json").read_text())
DT = {"f32": F32, "bf16": BF16, "q8_0": Q8_0, "q4_0": Q4_0, "mxfp4": MXFP4}
E2M1X2 = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
QUANT = [Q8_0, Q4_0, MXFP4]


def f16(u16):
    return float(np.array([u16], np.uint16).view(np.float16)[0])


def block_values(dtype, raw):
    """One ggml block -> its 32 values in float64 from the format's definition (model.h:58-60,
    kernels.h:20): q8_0 q*d, q4_0 (n-8)*d with byte i = (x[i] low, x[i+16] high), mxfp4 e2m1(n)*2^(e-127)/2."""
    raw = bytes(raw)
    if dtype == Q8_0:
        d = f16(int.from_bytes(raw[:2], "little"))
        return np.array([d * v for v in np.frombuffer(raw[2:], np.int8)], np.float64)
    nib = raw[2:] if dtype == Q4_0 else raw[1:]
    codes = [b & 15 for b in nib] + [b >> 4 for b in nib]
    if dtype == Q4_0:
        d = f16(int.from_bytes(raw[:2], "little"))
        return np.array([d * (c - 8) for c in codes], np.float64)
    return np.array([2.0 ** (raw[0] - 128) * E2M1X2[c] for c in codes], np.float64)


# ------------------------------------------------------------------------ golden vectors of the reference

@pytest.mark.parametrize("case", BLOCKS["ggml"], ids=lambda c: f"{c['dtype']}-{c['input']}")
def test_quantizer_matches_ggml_golden_bytes(case):
    """The generator's quantizer (it writes every benchmark model) reproduces ggml's bytes, ties included."""
    x = np.float32(BLOCKS["inputs"][case["input"]])
    got = A.quantize_rows(DT[case["dtype"]], x[None, :])[0].tobytes().hex()
    assert got == case["hex"]


def test_q8_0_rounds_by_the_reciprocal():
    c = BLOCKS["q8_0_reciprocal"]
    raw = A.quantize_rows(Q8_0, np.float32(c["x"])[None, :])[0]
    assert int(raw[2:].view(np.int8)[c["index"]]) == c["q"]


@pytest.mark.parametrize("case", BLOCKS["ggml"], ids=lambda c: f"{c['dtype']}-{c['input']}")
def test_oracle_dequant_of_golden_blocks(oracle, case):
    """Exact unpacking (pack.c:55-62) of the golden blocks: the oracle equals the block definition."""
    raw = np.frombuffer(bytes.fromhex(case["hex"]), np.uint8)
    got = oracle.dequant(DT[case["dtype"]], raw[None, :], 32)[0]
    np.testing.assert_array_equal(got.astype(np.float64), block_values(DT[case["dtype"]], raw))


def test_bf16_round_to_nearest_even(oracle):
    c = BLOCKS["bf16_rne"]
    got = [oracle.lib.or_bf16_f32(oracle.lib.or_f32_bf16(v)) for v in np.float32(c["x"])]
    assert got == c["expect"]
    np.testing.assert_array_equal(to_bf16(np.float32(c["x"])), [oracle.lib.or_f32_bf16(v) for v in np.float32(c["x"])])


def test_f16_decode_exhaustive(oracle):
    """All 65536 halves, subnormals, infinities and NaN payloads included, against numpy's float16."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib.or_f16_f32(int(v)) for v in h], np.float32)
    fin = np.isfinite(want)
    np.testing.assert_array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_f16_encode_matches_numpy():
    """The generator's f32 -> f16 (block scales): round to nearest even, subnormals, overflow to inf."""
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(20000) * s for s in (1e-8, 1e-6, 1e-4, 1e-2, 1, 100, 3e4, 7e4)]).astype(np.float32)
    x = np.concatenate([x, np.float32([0, -0.0, 65504, 65520, 65519.99, 2 ** -24, 2 ** -25, 2 ** -26, 3 * 2 ** -26, np.inf, -np.inf])])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([A.lib().l3m_f32_to_f16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", QUANT + [BF16, F32])
def test_dequant_rows_match_block_definition(oracle, dtype):
    k = 96
    r = extremes(dtype, rows(dtype, 5, k, seed=11), k)
    got = oracle.dequant(dtype, r, k).astype(np.float64)
    if dtype == F32:
        want = r.view(np.float32).astype(np.float64)
    elif dtype == BF16:
        want = (r.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    else:
        bb = {Q8_0: 34, Q4_0: 18, MXFP4: 17}[dtype]
        want = np.array([np.concatenate([block_values(dtype, row[b * bb:(b + 1) * bb]) for b in range(k // 32)]) for row in r])
    np.testing.assert_array_equal(got, want)


# ----------------------------------------------------------------------------- activation prep and gemv

@pytest.mark.parametrize("n", [32, 96, 768])
def test_prepare_invariants(oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32) * 3
    x[:32] = 0                                   # an all-zero block: scale 0, codes 0
    p = oracle.prepare(Q8_0, x)
    q, scale, s = p["q8"].astype(np.int64), p["scale"], p["sum"]
    assert np.abs(q).max() <= 127
    np.testing.assert_array_equal(s, q.reshape(-1, 32).sum(axis=1))
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    np.testing.assert_array_equal(scale, (amax / np.float32(127)).astype(np.float32))
    blocks = q.reshape(-1, 32)
    assert all(np.abs(blocks[b]).max() == 127 for b in range(len(blocks)) if amax[b] > 0)
    assert not blocks[0].any()
    # every code is the nearest integer to x * 127/amax (ties away from zero do not occur in random data)
    mul = np.divide(127.0, amax, out=np.zeros(len(amax)), where=amax > 0)
    xs = x.reshape(-1, 32).astype(np.float64) * mul[:, None]
    assert np.abs(blocks - xs).max() <= 0.5 + 1e-5


@pytest.mark.parametrize("dtype", [BF16] + QUANT)
@pytest.mark.parametrize("n", [32, 288, 768])
def test_prepare_matches_reference(oracle, reference, dtype, n):
    x = np.random.default_rng(n + dtype).standard_normal(n).astype(np.float32)
    x[5] = 0
    x[40 % n] = -3.5
    mine = oracle.prepare(dtype, x)
    v, keep = reference.prepare(dtype, x)
    if dtype == BF16:
        np.testing.assert_array_equal(mine["bf16"], np.ctypeslib.as_array(v.bf16, (n,)))
        return
    np.testing.assert_array_equal(mine["q8"], np.ctypeslib.as_array(v.q8, (n,)))
    np.testing.assert_array_equal(mine["scale"], np.ctypeslib.as_array(v.scale, (n // 32,)))
    np.testing.assert_array_equal(mine["sum"], np.ctypeslib.as_array(v.sum, (n // 32,)))


@pytest.mark.parametrize("dtype", [F32, BF16] + QUANT)
@pytest.mark.parametrize("shape", [(48, 288), (32, 768), (17, 64)])
def test_gemv_matches_reference_scalar_bit_exact(oracle, reference, dtype, shape):
    n, k = shape
    r = extremes(dtype, rows(dtype, n, k, seed=n * k + dtype), k)
    x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
    tiles = reference.pack_tiles(dtype, list(r) + [None] * (-n % 16), k)
    want = reference.gemv("scalar", dtype, tiles, (n + 15) // 16, k, x)[:n]
    got = oracle.gemv(dtype, r, n, k, x)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", [F32, BF16] + QUANT)
def test_gemv_close_to_float64(oracle, dtype):
    """Against float64 over the exactly unpacked weights and the prepared activation (test_kernels.c:114)."""
    n, k = 64, 768
    r = rows(dtype, n, k, seed=3)
    x = np.random.default_rng(4).standard_normal(k).astype(np.float32)
    w = oracle.dequant(dtype, r, k).astype(np.float64)
    if dtype == F32:
        xp = x.astype(np.float64)
    elif dtype == BF16:
        xp = (to_bf16(x).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    else:
        p = oracle.prepare(dtype, x)
        xp = (p["q8"].reshape(-1, 32).astype(np.float64) * p["scale"][:, None]).ravel()
    want = w @ xp
    got = oracle.gemv(dtype, r, n, k, x).astype(np.float64)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(w).sum(axis=1).max() * np.abs(xp).max()


# ------------------------------------------------------------------------------------------ ops

def test_rmsnorm_close_to_float64(oracle):
    x = np.random.default_rng(1).standard_normal(768).astype(np.float32)
    w = (1 + 0.1 * np.random.default_rng(2).standard_normal(768)).astype(np.float32)
    want = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5) * w
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-5), want, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("pos", [0, 1, 77])
def test_rope_close_to_float64(oracle, pos):
    hd, nh = 64, 3
    v = np.random.default_rng(pos).standard_normal(nh * hd).astype(np.float32)
    i = np.arange(hd // 2)
    ang = pos * 10000.0 ** (-2.0 * i / hd)
    a, b = v.reshape(nh, hd // 2, 2)[..., 0].astype(np.float64), v.reshape(nh, hd // 2, 2)[..., 1].astype(np.float64)
    want = np.stack([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], -1).ravel()
    np.testing.assert_allclose(oracle.rope(v, nh, hd, pos, 10000.0), want, rtol=1e-4, atol=1e-5)
    if pos == 0:                                  # angle 0: the identity, exactly
        np.testing.assert_array_equal(oracle.rope(v, nh, hd, 0, 10000.0), v)


def test_silu_mul_close_to_float64(oracle):
    h, g = (np.random.default_rng(s).standard_normal(512).astype(np.float32) * 4 for s in (1, 2))
    want = h.astype(np.float64) * g / (1 + np.exp(-g.astype(np.float64)))
    np.testing.assert_allclose(oracle.silu_mul(h, g), want, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("pos,hd", [(0, 48), (9, 64), (200, 64)])
def test_attend_close_to_float64(oracle, pos, hd):
    """test_kernels.c:124-149: softmax attention against float64 within 1e-5."""
    rng = np.random.default_rng(pos + hd)
    stride = hd * 3
    q = rng.standard_normal(hd).astype(np.float32)
    k = to_bf16(rng.standard_normal((pos + 1) * stride))
    v = to_bf16(rng.standard_normal((pos + 1) * stride))
    kf = (k.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(pos + 1, stride)[:, :hd]
    vf = (v.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(pos + 1, stride)[:, :hd]
    s = kf @ q.astype(np.float64) / np.sqrt(hd)
    p = np.exp(s - s.max())
    want = (p / p.sum()) @ vf
    np.testing.assert_allclose(oracle.attend(q, k, v, pos, hd, stride), want, atol=1e-5)


@pytest.mark.parametrize("pos,hd", [(0, 48), (37, 64), (255, 64)])
def test_attend_matches_reference_scalar_bit_exact(oracle, reference, pos, hd):
    rng = np.random.default_rng(pos * hd)
    stride = hd * 2
    q = rng.standard_normal(hd).astype(np.float32)
    k, v = to_bf16(rng.standard_normal((pos + 1) * stride)), to_bf16(rng.standard_normal((pos + 1) * stride))
    np.testing.assert_array_equal(oracle.attend(q, k, v, pos, hd, stride), reference.attend("scalar", q, k, v, pos, hd, stride))


# ------------------------------------------------------------------------------------ engine

def sha(path):
    return hashlib.sha256(path.read_bytes()).hexdigest()


def logits_summary_sha(lg):
    return hashlib.sha256(np.ascontiguousarray(lg, np.float32).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def cases(golden, models):
    return {(c["config"], c["dtype"]): (c, models.get(c["config"], c["dtype"])) for c in golden["cases"]}


@pytest.mark.parametrize("key", [("stories15M", "bf16"), ("stories42M", "q8_0"), ("stories110M", "q4_0"),
                                 ("smollm2", "q8_0"), ("smollm2", "mxfp4")], ids=lambda k: f"{k[0]}-{k[1]}")
def test_generator_and_oracle_engine_match_golden(oracle, cases, key):
    """The seeded model bytes are the ones the golden run used, and the oracle engine reproduces the
    reference's scalar engine bit for bit: prompt logits (SHA-256) and the greedy tokens."""
    case, path = cases[key]
    assert sha(path) == case["sha256"]
    cfg = A.CONFIGS[case["config"]]
    assert A.prompt(1, cfg.vocab, cfg.n_prompt) == case["prompt"]
    om = oracle.load(path)
    om.generate(case["prompt"], 0)
    assert logits_summary_sha(om.logits()) == case["scalar_prompt_logits"]["sha256"]
    n = 64 if cfg.n_layers * cfg.dim <= 12 * 768 else 16
    assert om.generate(case["prompt"], n) == case["scalar_tokens"][:n]


@pytest.mark.parametrize("key", [("stories15M", "bf16"), ("stories110M", "q4_0")], ids=lambda k: f"{k[0]}-{k[1]}")
def test_oracle_reference_mode_matches_golden(oracle, cases, key):
    """The fp32 oracle path (ref.c:98-143) equals the reference's --ref prompt logits bit for bit."""
    case, path = cases[key]
    om = oracle.load(path, ref=True)
    om.generate(case["prompt"], 0)
    assert logits_summary_sha(om.logits()) == case["ref_prompt_logits"]["sha256"]
