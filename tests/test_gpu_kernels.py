"""Parity of each device kernel, called through the C ABI, against the CPU oracle on the same seeded inputs.

Bars: bit-exact activation quantization and block unpacking; matvec within 1e-3 relative
(bf16, q8_0, f32) or 5e-3 (q4_0, mxfp4) of the oracle, relative to max|y|; attention within 1e-5 absolute of
the oracle (the reference's own bar vs double, tests/test_kernels.c:145).
"""
import numpy as np
import pytest

from weights import BF16, F32, MXFP4, Q4_0, Q8_0, SHAPES, extremes, rel_err, rows

pytestmark = pytest.mark.gpu
TOL = {F32: 1e-3, BF16: 1e-3, Q8_0: 1e-3, Q4_0: 5e-3, MXFP4: 5e-3}
NAMES = {F32: "f32", BF16: "bf16", Q8_0: "q8_0", Q4_0: "q4_0", MXFP4: "mxfp4"}


def split_act(raw, k):
    kp = (k + 31) // 32 * 32
    nb = kp // 32
    return raw[:k].view(np.int8), raw[kp:kp + 4 * nb].view(np.float32), raw[kp + 4 * nb:kp + 8 * nb].view(np.int32)


@pytest.mark.parametrize("k", [32, 288, 768, 1376, 2048, 4096])
def test_prep_quantized_bit_exact(dev, oracle, k):
    rng = np.random.default_rng(k)
    x = rng.standard_normal(k).astype(np.float32) * 3
    x[:32] = 0                                        # an all-zero block: scale 0, inv 0
    if k > 64:
        x[40] = 1e-30                                 # tiny values around a large one
        x[64:96] = np.float32(0.5) * np.arange(32) - 8   # exact .5 products: rint ties to even
    q8, scale, s = split_act(dev.prep(Q8_0, x), k)
    want = oracle.prepare(Q8_0, x)
    assert np.array_equal(q8, want["q8"])
    assert np.array_equal(scale.view(np.uint32), want["scale"].view(np.uint32))
    assert np.array_equal(s, want["sum"])


def fp8_e4m3(b):
    """Values of fp8 e4m3 bytes (no NaN among the bytes checked here)."""
    b = np.asarray(b, np.int64)
    e, m = (b >> 3) & 15, b & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7))
    return np.where(b & 0x80, -v, v)


@pytest.mark.parametrize("k", [32, 288, 1376, 4096])
def test_prep_mxfp4_parts(dev, oracle, k):
    """The mxfp4 form: f16 pairs (q[j], q[j + 16]) per block, the scales and sums, then per block the fp8
    parts h = floor(q / 16) and l = q - 16 h of the pairs' elements (the matrix-core matvec's operand)."""
    rng = np.random.default_rng(k + 9)
    x = rng.standard_normal(k).astype(np.float32) * 3
    x[:32] = 0
    if k > 64:
        x[40] = -12.0                                 # the block's largest: q = -127
    raw = dev.prep(MXFP4, x)
    nb = (k + 31) // 32
    want = oracle.prepare(Q8_0, x)
    q = np.zeros(nb * 32, np.int64)
    q[:k] = want["q8"]
    q = q.reshape(nb, 32)
    pairs = raw[:64 * nb].view(np.float16).reshape(nb, 16, 2)
    elem = np.stack([q[:, :16], q[:, 16:]], axis=2)  # element e = 2j + i: q[j + 16 i]
    assert np.array_equal(pairs.astype(np.int64), elem)
    assert np.array_equal(raw[64 * nb:68 * nb].view(np.float32).view(np.uint32), want["scale"].view(np.uint32))
    hl = raw[72 * nb:136 * nb].reshape(nb, 2, 32)
    assert len(raw) == 136 * nb
    e = elem.reshape(nb, 32)
    assert np.array_equal(fp8_e4m3(hl[:, 0]), np.floor(e / 16))
    assert np.array_equal(fp8_e4m3(hl[:, 1]), e - 16 * np.floor(e / 16))


@pytest.mark.parametrize("k", [2, 18, 288, 4096])
def test_prep_bf16_bit_exact(dev, oracle, k):
    x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
    raw = dev.prep(BF16, x)
    assert np.array_equal(raw[: 2 * k].view(np.uint16), oracle.prepare(BF16, x)["bf16"])


@pytest.mark.parametrize("dtype", [F32, BF16, Q8_0, Q4_0, MXFP4], ids=NAMES.get)
@pytest.mark.parametrize("shape", SHAPES[:3], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_small_shapes(dev, oracle, dtype, shape):
    n, k = shape
    w = rows(dtype, n, k, seed=n + k + dtype)
    x = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    y = dev.gemv(dev.matrix(dtype, w, k), x)
    want = oracle.gemv(dtype, w, n, k, x)
    assert rel_err(y, want) < TOL[dtype], rel_err(y, want)
    dev.free_all()


@pytest.mark.parametrize("dtype", [BF16, Q8_0, Q4_0, MXFP4], ids=NAMES.get)
@pytest.mark.parametrize("shape", SHAPES[3:], ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_large_shapes(dev, oracle, dtype, shape):
    n, k = shape
    w = rows(dtype, n, k, seed=7)
    x = np.random.default_rng(2).standard_normal(k).astype(np.float32)
    y = dev.gemv(dev.matrix(dtype, w, k), x)
    want = oracle.gemv(dtype, w, n, k, x)
    assert rel_err(y, want) < TOL[dtype], rel_err(y, want)
    dev.free_all()


@pytest.mark.parametrize("dtype", [Q8_0, Q4_0, MXFP4], ids=NAMES.get)
@pytest.mark.parametrize("k", [288, 1376, 3072])
def test_gemv_edges(dev, oracle, dtype, k):
    """q8 weight -128, subnormal mxfp4 scales, a zero activation block, zero (missing) rows."""
    n = 48
    w = extremes(dtype, rows(dtype, n, k, seed=k), k)
    w_list = [w[i] if i < n - 5 else None for i in range(n)]
    x = np.random.default_rng(3).standard_normal(k).astype(np.float32) * 4
    x[:32] = 0
    y = dev.gemv(dev.matrix(dtype, w_list, k), x)
    w0 = w.copy()
    w0[n - 5:] = 0
    want = oracle.gemv(dtype, w0, n, k, x)
    want[n - 5:] = 0
    assert np.all(y[n - 5:] == 0)
    assert rel_err(y, want) < TOL[dtype], rel_err(y, want)
    dev.free_all()


@pytest.mark.parametrize("dtype", [Q8_0, Q4_0, MXFP4], ids=NAMES.get)
@pytest.mark.parametrize("k", [2048, 4096, 8192])
def test_gemv_deep_edges(dev, oracle, dtype, k):
    """The same extremes on the shapes of the 8-wavefront matvecs (at least 128 tiles, rows of 64, 128 or 256
    blocks; mxfp4 on the matrix cores): a q8 weight of -128 and subnormal mxfp4 scales in every block, a zero
    activation block, an activation of one large value in a block (q = +-127 there), and a ragged last tile."""
    n = 2048 + 5
    w = extremes(dtype, rows(dtype, n, k, seed=k + 1), k)
    x = np.random.default_rng(5).standard_normal(k).astype(np.float32)
    x[:32] = 0
    x[64:96] = -1e-3
    x[70] = -50.0
    x[100] = 50.0
    y = dev.gemv(dev.matrix(dtype, w, k), x)
    want = oracle.gemv(dtype, w, n, k, x)
    assert rel_err(y, want) < TOL[dtype], rel_err(y, want)
    dev.free_all()


@pytest.mark.parametrize("k", [4096])
def test_gemv_mxfp4_matrix_cores_equal_valu_dots(dev, oracle, k):
    """The matrix-core mxfp4 matvec gives the VALU form's results bit for bit at 128 blocks per row (the same
    per-block values, the same split over 8 wavefronts and order of additions), extremes included, and
    meets the oracle. (At 64 blocks per row the two forms split a tile differently; at 256 the VALU form's
    activation does not fit the 8-wavefront kernel's staging and the 4-wavefront kernel runs.)"""
    n = 2048 + 16 * 3
    w = extremes(MXFP4, rows(MXFP4, n, k, seed=k + 3), k)
    w[::7] = rows(MXFP4, n, k, seed=k + 4)[::7]          # ordinary scales on every 7th row
    x = np.random.default_rng(6).standard_normal(k).astype(np.float32)
    x[32:64] = 0
    m = dev.matrix(MXFP4, w, k)
    was = dev.lib.l3m_gemv_matrix_cores(1)
    try:
        y_mx = dev.gemv(m, x)
        dev.lib.l3m_gemv_matrix_cores(0)
        y_valu = dev.gemv(m, x)
    finally:
        dev.lib.l3m_gemv_matrix_cores(was)
    assert np.array_equal(y_mx.view(np.uint32), y_valu.view(np.uint32))
    want = oracle.gemv(MXFP4, w, n, k, x)
    assert rel_err(y_mx, want) < TOL[MXFP4], rel_err(y_mx, want)
    dev.free_all()


@pytest.mark.parametrize("dtype,k", [(F32, 2), (F32, 18), (F32, 34), (BF16, 2), (BF16, 18), (BF16, 34)])
def test_gemv_ragged_k(dev, oracle, dtype, k):
    n = 33
    w = rows(dtype, n, k, seed=k)
    x = np.random.default_rng(4).standard_normal(k).astype(np.float32)
    y = dev.gemv(dev.matrix(dtype, w, k), x)
    assert rel_err(y, oracle.gemv(dtype, w, n, k, x)) < TOL[dtype]
    dev.free_all()


@pytest.mark.parametrize("hd", [16, 32, 40, 48, 64])
@pytest.mark.parametrize("pos", [0, 1, 37, 255])
def test_attend(dev, oracle, hd, pos):
    rng = np.random.default_rng(hd * 1000 + pos)
    stride = 3 * hd
    q = (rng.standard_normal(hd) * 2).astype(np.float32)
    k = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBFFF   # bf16 with |v| < 2
    v = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBFFF
    got = dev.attend(q, k, v, pos, hd, stride)
    want = oracle.attend(q, k, v, pos, hd, stride)
    assert np.abs(got - want).max() <= 1e-5
    dev.free_all()


def test_attend_large_scores(dev, oracle):
    """qscale 40 pushes scores far past exp's range (tests/test_kernels.c:197)."""
    rng = np.random.default_rng(40)
    hd, pos, stride = 64, 255, 192
    q = (rng.uniform(-1, 1, hd) * 40).astype(np.float32)
    k = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBF7F
    v = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBF7F
    assert np.abs(dev.attend(q, k, v, pos, hd, stride) - oracle.attend(q, k, v, pos, hd, stride)).max() <= 1e-5
    dev.free_all()


@pytest.mark.parametrize("n", [64, 288, 576, 768])
def test_rmsnorm(dev, oracle, n):
    rng = np.random.default_rng(n)
    x, w = rng.standard_normal(n).astype(np.float32), (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    assert rel_err(dev.rmsnorm(x, w, 1e-5), oracle.rmsnorm(x, w, 1e-5)) < 1e-6


@pytest.mark.parametrize("hd,pos", [(48, 0), (48, 7), (64, 127), (64, 1023)])
def test_rope(dev, oracle, hd, pos):
    n_heads = 6
    v = np.random.default_rng(pos).standard_normal(n_heads * hd).astype(np.float32)
    got = dev.rope(v, n_heads, hd, pos, 10000.0)
    want = oracle.rope(v, n_heads, hd, pos, 10000.0)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_silu_mul(dev, oracle):
    rng = np.random.default_rng(5)
    h, g = rng.standard_normal(2048).astype(np.float32), (rng.standard_normal(2048) * 4).astype(np.float32)
    assert rel_err(dev.silu_mul(h, g), oracle.silu_mul(h, g)) < 1e-6


def test_argmax_lowest_index_wins(dev):
    x = np.random.default_rng(6).standard_normal(49152).astype(np.float32)
    assert dev.argmax(x) == int(np.argmax(x))
    x[[100, 7000, 40000]] = x.max() + 1
    assert dev.argmax(x) == 100
    assert dev.argmax(np.zeros(32000, np.float32)) == 0
    dev.free_all()


@pytest.mark.parametrize("dtype", [F32, BF16, Q8_0, Q4_0, MXFP4], ids=NAMES.get)
def test_table_matches_reference_tables(reference, dtype):
    """l3m_kernels_hip on the reference's own packed tiles and prepared vector, against its scalar table; the
    128-tile case takes the 8-wavefront matvecs (mxfp4 on the matrix cores, from the table's own prepared
    form)."""
    import ctypes as C
    import l3m_amd as A
    from oracle.oracle import _Table
    lib = A.lib()
    table = _Table.in_dll(lib, "l3m_kernels_hip")
    assert table.name == b"hip"
    for k, ntiles in [(288, 3), (1376, 2), (3072, 5), (4096, 128)]:
        n = ntiles * 16
        w = rows(dtype, n, k, seed=k + dtype)
        tiles = reference.pack_tiles(dtype, [w[i] if i < n - 3 else None for i in range(n)], k)
        x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
        v, keep = reference.prepare(dtype, x)
        y = np.zeros(n, np.float32)
        table.gemv[dtype](y.ctypes.data_as(C.POINTER(C.c_float)), tiles.ctypes.data, ntiles, k, C.byref(v))
        want = reference.gemv("scalar", dtype, tiles, ntiles, k, x)
        assert rel_err(y, want) < TOL[dtype], (k, rel_err(y, want))


@pytest.mark.parametrize("hd,pos,stride", [(64, 100, 128), (48, 0, 48), (32, 1, 96), (128, 511, 128), (64, 4000, 64)])
def test_table_attend_matches_reference(reference, hd, pos, stride):
    """The table's attend (kernels.h: one query head over rows 0..pos of K and V with a row stride) against
    the reference's scalar table, 1e-5 absolute (tests/test_kernels.c:145): head dims 32 to 128, the first
    position, the second, and 4,001 positions."""
    import ctypes as C
    import l3m_amd as A
    from oracle.oracle import _Table
    table = _Table.in_dll(A.lib(), "l3m_kernels_hip")
    rng = np.random.default_rng(9 + hd + pos)
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBFFF
    v = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBFFF
    out = np.zeros(hd, np.float32)
    f, u16 = C.POINTER(C.c_float), C.POINTER(C.c_uint16)
    table.attend(out.ctypes.data_as(f), q.ctypes.data_as(f), k.ctypes.data_as(u16), v.ctypes.data_as(u16), pos, hd, stride)
    assert np.abs(out - reference.attend("scalar", q, k, v, pos, hd, stride)).max() <= 1e-5


@pytest.mark.parametrize("dtype", [F32, BF16, Q8_0, Q4_0, MXFP4], ids=NAMES.get)
@pytest.mark.parametrize("k", [288, 1376])
def test_dequant_bit_exact(dev, oracle, dtype, k):
    """The decode step's device dequantization (lt_elem4: the embedding lookup, engine.c:236) against the
    reference's l3m_dequant_row restated (pack.c:55-62), bit for bit, including the values the quantizers
    never make (q8 -128, subnormal mxfp4 scales) and zero rows."""
    n = 40
    w = rows(dtype, n, k, seed=k + 10 * dtype)
    if dtype in (Q8_0, MXFP4):
        w = extremes(dtype, w, k)
    w_list = [w[i] if i < n - 3 else None for i in range(n)]
    m = dev.matrix(dtype, w_list, k)
    got = dev.dequant(m, 0, n)
    w0 = w.copy()
    w0[n - 3:] = 0
    want = oracle.dequant(dtype, w0, k)
    assert np.array_equal(got[:, :k].view(np.uint32), want.view(np.uint32))
    assert not got[:, k:].any()
    part = dev.dequant(m, 17, 5)                      # a row range inside and across tiles
    assert np.array_equal(part[:, :k].view(np.uint32), want[17:22].view(np.uint32))
    dev.free_all()
