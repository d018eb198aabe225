"""The decode step's own attention (the code attn_block runs, through l3m_k_attend_decode), in each of its
three forms, against the oracle's l3m_attend (ops.c:42-73) per query head, within 1e-5 absolute: the
reference's own bar against double precision (tests/test_kernels.c:145).

  mode 2  attend_mfma: scores and P.V on the matrix cores, q and p split into three bf16 parts
  mode 1  attend_group over the K/V window in LDS (head dims that are not a multiple of 16)
  mode 0  attend_group reading K and V from the cache (windows too long for LDS)

Positions cover the 16-position tiles and 32-position steps of mode 2 and the split-softmax rounds of
modes 0 and 1 (0, 1, 15, 16, 63, 64, 127, 255, 511, 600), at q scales 1 and 40 (40 pushes scores far past
expf's range, tests/test_kernels.c:197), for one query head per kv head, two, and grouped heads.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
POSITIONS = [0, 1, 15, 16, 63, 64, 127, 255, 511, 600]


def inputs(seed, nq, nkv, hd, ctx, qscale):
    rng = np.random.default_rng(seed)
    q = (rng.uniform(-1, 1, (nq, hd)) * qscale).astype(np.float32)
    kc = (rng.integers(0, 1 << 16, (nkv, ctx, hd), dtype=np.uint16) & 0xBF7F).astype(np.uint16)   # bf16, |v| < 2
    vc = (rng.integers(0, 1 << 16, (nkv, ctx, hd), dtype=np.uint16) & 0xBF7F).astype(np.uint16)
    return q, kc, vc


def want(oracle, q, kc, vc, nq, nkv, hd, pos):
    hpk = nq // nkv
    return np.stack([oracle.attend(q[h], kc[h // hpk].ravel(), vc[h // hpk].ravel(), pos, hd, hd) for h in range(nq)])


# (mode, hd, nq, nkv, ctx): the window of modes 1 and 2 must fit in LDS beside the rest, so their ctx is
# the largest that does for the shape; mode 0 takes the longest positions.
CASES = [(2, 64, 1, 1, 512), (2, 64, 2, 1, 320), (2, 48, 1, 1, 512), (2, 48, 2, 2, 256), (2, 48, 2, 1, 512), (2, 32, 1, 1, 512),
         (2, 80, 1, 1, 256), (2, 80, 2, 1, 256), (1, 64, 1, 1, 512), (1, 48, 2, 2, 256), (1, 48, 2, 1, 512),
         (0, 64, 1, 1, 1024), (0, 48, 2, 2, 1024), (0, 64, 3, 1, 1024), (0, 32, 1, 1, 1024)]


@pytest.mark.parametrize("qscale", [1.0, 40.0])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"mode{c[0]}-hd{c[1]}-nq{c[2]}-nkv{c[3]}")
def test_decode_attention_matches_oracle(dev, oracle, case, qscale):
    mode, hd, nq, nkv, ctx = case
    worst = 0.0
    for pos in POSITIONS:
        if pos >= ctx:
            continue
        print(f"attention mode {mode} hd {hd} nq {nq} nkv {nkv} ctx {ctx} pos {pos} qscale {qscale}", flush=True)
        q, kc, vc = inputs(1000 * hd + pos + int(qscale), nq, nkv, hd, ctx, qscale)
        got = dev.attend_decode(mode, q, kc, vc, nq, nkv, hd, ctx, pos)
        err = float(np.abs(got - want(oracle, q, kc, vc, nq, nkv, hd, pos)).max())
        worst = max(worst, err)
        assert err <= 1e-5, (pos, err)
        dev.free_all()
    print(f"worst |gpu - oracle| {worst:.2e}", flush=True)


def test_attention_modes_agree_with_decode_choice(dev):
    """The mode a decode step picks (l3m_attention_mode) for the benchmark shapes: matrix cores for hd 64
    and 48 with the window in LDS, the VALU window form for a head dimension off the multiples of 16, the
    cache form without a window."""
    import l3m_amd as A
    lib = A.lib()
    assert lib.l3m_attention_mode(1, 64, 1, 128) == 2
    assert lib.l3m_attention_mode(1, 48, 2, 256) == 2
    assert lib.l3m_attention_mode(1, 40, 2, 256) == 1
    assert lib.l3m_attention_mode(0, 64, 1, 1024) == 0
    assert lib.l3m_attention_mode(1, 64, 12, 128) == 1    # too many heads' q parts beside the sums
