"""The decode step's own matvecs, one matrix at a time, at the north star's per-kernel bars.

The decode step does not run the microbench's k_gemv: it streams each layer's matrices as head groups
(q/k/v rows and Wo columns) and FFN chunks (gate/up rows and Wdown columns), q4_0 bodies (and mxfp4 bodies
whose block scales are f16 powers of two) widened at load to q8_0 blocks of the same values, through three
forms (tile_rows for the quantized wide matrices and the head, slots_rows or mv with rows_sum4 for the
column slices, mv with rows_sum4 for bf16). l3m_step_matvec runs one stored matrix of a loaded model
through exactly the device code the step runs it with, the int8 prep of the input included, and each is
compared here with the oracle's gemv of the file's own rows (kernels_scalar.c:19-75, the reference's
per-block formula): within 1e-3 of max|y| for bf16 and q8_0 and 5e-3 for q4_0 and mxfp4 (the north star's
bars, tests/test_kernels.c:114 measures against double the same way). With the same prepared input the two
differ only in the order of the fp32 additions of block sums: the largest error measured over every group,
chunk and head of the first and last layers of all six cases is 4.4e-7 of max|y| (stories15M's head), so
the error is also held to 1e-6.
"""
import numpy as np
import pytest

import l3m_amd as A
from weights import read_tensors, rel_err

pytestmark = pytest.mark.gpu
TOL = {"f32": 1e-3, "bf16": 1e-3, "q8_0": 1e-3, "q4_0": 5e-3, "mxfp4": 5e-3}
ORDER_ONLY = 1e-6
CASES = [("stories15M", "bf16", None), ("stories42M", "q8_0", None), ("stories110M", "q4_0", None),
         ("smollm2", "q8_0", None), ("smollm2", "mxfp4", None), ("smollm2", "mxfp4", "0")]


def cols(rows, dtype, c0, c1):
    """Columns [c0, c1) of file rows (whole 32-blocks for quantized rows)."""
    per = {A.F32: 4, A.BF16: 2}
    if dtype in per:
        return rows[:, per[dtype] * c0:per[dtype] * c1]
    bb = A.BLOCK_BYTES[dtype]
    return rows[:, c0 // 32 * bb:c1 // 32 * bb]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}" + ("-e2m1" if c[2] else ""))
def test_step_matvecs_match_oracle(models, oracle, monkeypatch, case):
    name, dtype, widen = case
    if widen is not None:
        monkeypatch.setenv("L3M_WIDEN", widen)
    path = models.get(name, dtype)
    print(f"step matvec: {name} {dtype} L3M_WIDEN={widen}", flush=True)
    t, d = read_tensors(path)
    m = A.Model(path)
    lay = m.step_layout()
    hd, dim, ffn = d["dim"] // d["n_heads"], d["dim"], d["ffn_dim"]
    hpk = d["n_heads"] // d["n_kv_heads"]
    dt = A.DTYPES[dtype]
    rng = np.random.default_rng(len(name) + dt)
    worst = {}

    def check(what, y, want):
        e = rel_err(y, want)
        worst[what] = max(worst.get(what, 0.0), e)
        assert e < TOL[dtype] and e < ORDER_ONLY, (what, e)

    for layer in sorted({0, d["n_layers"] - 1}):
        L = lambda n: t[f"blk.{layer}.{n}"][2]
        for g in range(lay["groups"]):
            q0, nq = g * lay["nq"], lay["nq"]
            kv0, kv1 = q0 // hpk, (q0 + nq - 1) // hpk + 1
            w = np.concatenate([L("wq")[q0 * hd:(q0 + nq) * hd], L("wk")[kv0 * hd:kv1 * hd], L("wv")[kv0 * hd:kv1 * hd]])
            x = rng.standard_normal(dim).astype(np.float32)
            check("qkv", m.step_matvec(0, layer, g, x, len(w)), oracle.gemv(dt, w, len(w), dim, x))
            wo = np.ascontiguousarray(cols(L("wo"), dt, q0 * hd, (q0 + nq) * hd))
            xo = rng.standard_normal(nq * hd).astype(np.float32)
            check("wo", m.step_matvec(1, layer, g, xo, dim), oracle.gemv(dt, wo, dim, nq * hd, xo))
        for c in range(lay["chunks"]):
            f0 = c * lay["chunk"]
            nf = min(lay["chunk"], ffn - f0)
            gu = np.zeros((2 * nf, L("w_gate").shape[1]), np.uint8)
            gu[0::2], gu[1::2] = L("w_gate")[f0:f0 + nf], L("w_up")[f0:f0 + nf]
            rows_gu = 32 * ((nf + 15) // 16)
            x = rng.standard_normal(dim).astype(np.float32)
            y = m.step_matvec(2, layer, c, x, rows_gu)
            assert not y[2 * nf:].any()                # the chunk's padding rows
            check("gate_up", y[:2 * nf], oracle.gemv(dt, gu, 2 * nf, dim, x))
            wd = np.ascontiguousarray(cols(L("w_down"), dt, f0, f0 + nf))
            xd = rng.standard_normal(nf).astype(np.float32)
            check("down", m.step_matvec(3, layer, c, xd, dim), oracle.gemv(dt, wd, dim, nf, xd))
    head = t["embed"][2]
    x = rng.standard_normal(dim).astype(np.float32)
    check("head", m.step_matvec(4, 0, 0, x, d["vocab"]), oracle.gemv(dt, head, d["vocab"], dim, x))
    print(f"step matvec: {name} {dtype} layout {lay} describe {m.describe()!r}", flush=True)
    print("step matvec: worst rel err " + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()), flush=True)
    m.close()
