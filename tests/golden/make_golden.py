"""Writes tests/golden/decode.json: greedy tokens and last-prompt logits of the benchmark configurations,
computed by fpedd/l3m itself (oracle/_ref, built from the reference's sources) with its scalar kernel
table (L3M_ISA=scalar) and with its fp32 reference path (--ref semantics, reference=1).

Inputs are the seeded synthetic models of l3m_amd.write_model; their SHA-256 is recorded so a test can
prove it regenerated the same bytes. Run from the repository root after building:
    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
os.environ["L3M_ISA"] = "scalar"

import numpy as np  # noqa: E402

import l3m_amd as A  # noqa: E402
from oracle.oracle import Oracle, Reference  # noqa: E402

N_GEN = 64
CASES = [("stories15M", "bf16"), ("stories42M", "q8_0"), ("stories110M", "q4_0"), ("smollm2", "q8_0"), ("smollm2", "mxfp4")]


def sha256(path):
    return hashlib.sha256(Path(path).read_bytes()).hexdigest()


def summary(logits, k=8):
    top = np.argsort(-logits.astype(np.float64), kind="stable")[:k]
    return {"top_ids": top.tolist(), "top_vals": [float(logits[i]) for i in top], "argmax": int(np.argmax(logits)),
            "sum": float(logits.astype(np.float64).sum()), "absmax": float(np.abs(logits).max()),
            "sha256": hashlib.sha256(np.ascontiguousarray(logits, np.float32).tobytes()).hexdigest()}


def margins(oracle, path, prompt, tokens):
    """Before each generated token: the top-2 logit margin / max|logit| of the scalar engine, its two
    highest-scoring ids (first maximum first) and its logits, teacher-forced over prompt + tokens. The
    oracle is bit-exact with the reference's scalar engine (checked through the prompt-logits hash); each
    step's argmax must be the reference's token."""
    om = oracle.load(path)
    seq, out, top2, logits = list(prompt) + list(tokens), [], [], []
    for pos in range(len(seq) - 1):
        lg = om.forward(seq[pos], pos, logits=pos >= len(prompt) - 1)
        if lg is None:
            continue
        order = np.argsort(-lg.astype(np.float64), kind="stable")
        assert int(order[0]) == seq[pos + 1], "the oracle left the reference's tokens"
        lv = np.sort(lg.astype(np.float64))
        out.append(round(float((lv[-1] - lv[-2]) / np.abs(lv).max()), 6))
        top2.append([int(order[0]), int(order[1])])
        logits.append(lg)
    return out, top2, logits


def simd_teacher_forced(ref, path, prompt, tokens, scalar_logits):
    """The reference's SIMD table fed the scalar engine's tokens: per step its argmax, and the largest
    max|SIMD logit - scalar logit| / max|scalar logit| over the steps (its own activation-quantization
    spread on this model)."""
    m = ref.load(path)
    picks, spread = [], 0.0
    for k, ls in enumerate(scalar_logits):
        m.generate(list(prompt) + list(tokens[:k]), 0)
        la = m.logits()
        picks.append(int(np.argmax(la)))
        spread = max(spread, float(np.abs(la.astype(np.float64) - ls).max() / np.abs(ls).max()))
    del m
    return picks, round(spread, 6)


def main():
    ref, oracle = Reference(), Oracle()
    out = {"n_gen": N_GEN, "seed": 1, "prompt_seed": 1, "cases": []}
    with tempfile.TemporaryDirectory() as d:
        for name, dtype in CASES:
            cfg = A.CONFIGS[name]
            path = A.write_model(Path(d) / f"{name}-{dtype}.l3m", cfg, dtype=dtype, seed=1)
            prompt = A.prompt(1, cfg.vocab, cfg.n_prompt)
            case = {"config": name, "dtype": dtype, "sha256": sha256(path), "prompt": prompt}
            for mode, is_ref in (("scalar", False), ("ref", True)):
                m = ref.load(path, reference=is_ref)
                m.generate(prompt, 0)
                case[f"{mode}_prompt_logits"] = summary(m.logits())
                case[f"{mode}_tokens"] = m.generate(prompt, N_GEN)
                case[f"{mode}_last_logits"] = summary(m.logits())
                case[f"{mode}_describe"] = m.describe()
                del m
            case["scalar_margins"], case["scalar_top2"], scalar_logits = margins(oracle, path, prompt, case["scalar_tokens"])
            os.environ["L3M_ISA"] = "avx512" if ref.usable("avx512") else "avx2"
            m = ref.load(path)
            simd = m.generate(prompt, N_GEN)
            del m
            picks, case["simd_spread"] = simd_teacher_forced(ref, path, prompt, case["scalar_tokens"], scalar_logits)
            case["simd_tf_disagree"] = [k for k, (a, b) in enumerate(zip(picks, case["scalar_tokens"])) if a != b]
            os.environ["L3M_ISA"] = "scalar"
            case["simd_table"] = "avx512" if ref.usable("avx512") else "avx2"
            case["simd_agree"] = next((i for i, (a, b) in enumerate(zip(simd, case["scalar_tokens"])) if a != b), N_GEN)
            print(name, dtype, case["scalar_tokens"][:8], "ref agrees on", sum(a == b for a, b in zip(case["scalar_tokens"], case["ref_tokens"])),
                  "simd agrees on", case["simd_agree"], "min margin", min(case["scalar_margins"]), "simd spread", case["simd_spread"],
                  "simd teacher-forced disagrees at", case["simd_tf_disagree"], flush=True)
            out["cases"].append(case)
    (Path(__file__).parent / "decode.json").write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
