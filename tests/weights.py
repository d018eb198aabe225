"""Seeded weight rows in the .l3m file encodings (ggml blocks), as the kernel microbench specifies them
bf16 N(0, 0.02); q8_0 values uniform in [-127, 127] with an f16 scale |N(0,0.02)|/127;
q4_0 nibbles uniform with an f16 scale N(0,0.02)/8; mxfp4 nibbles uniform with e8m0 exponents in 119..123.
"""
import numpy as np

F32, BF16, Q8_0, Q4_0, MXFP4 = range(5)
ROW_BYTES = {F32: lambda k: 4 * k, BF16: lambda k: 2 * k, Q8_0: lambda k: k // 32 * 34, Q4_0: lambda k: k // 32 * 18,
             MXFP4: lambda k: k // 32 * 17}
SHAPES = [(288, 768), (768, 288), (2048, 768), (4096, 4096), (14336, 4096)]


def to_bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def rows(dtype, n, k, seed=0):
    rng = np.random.default_rng(seed)
    if dtype == F32:
        return (rng.standard_normal((n, k)) * 0.02).astype(np.float32).view(np.uint8).reshape(n, -1)
    if dtype == BF16:
        return to_bf16(rng.standard_normal((n, k)) * 0.02).view(np.uint8).reshape(n, -1)
    nb = k // 32
    if dtype == Q8_0:
        d = (np.abs(rng.standard_normal((n, nb))) * 0.02 / 127).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
        q = rng.integers(-127, 128, (n, nb, 32), dtype=np.int8).view(np.uint8)
        return np.concatenate([d, q], axis=2).reshape(n, -1)
    q = rng.integers(0, 256, (n, nb, 16), dtype=np.uint8)
    if dtype == Q4_0:
        d = (rng.standard_normal((n, nb)) * 0.02 / 8).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
        return np.concatenate([d, q], axis=2).reshape(n, -1)
    e = rng.integers(119, 124, (n, nb, 1), dtype=np.uint8)
    return np.concatenate([e, q], axis=2).reshape(n, -1)


def extremes(dtype, r, k):
    """Legal values the quantizers never make (the reference's tests/test_kernels.c:62-68): a q8 weight of
    -128 per block and subnormal mxfp4 scales e in {0, 1, 2}."""
    r = r.copy()
    for i in range(len(r)):
        for b in range(k // 32):
            if dtype == Q8_0:
                r[i, b * 34 + 2 + b % 32] = 0x80
            if dtype == MXFP4:
                r[i, b * 17] = (i + b) % 3
    return r


def rel_err(got, want):
    return float(np.abs(np.float64(got) - np.float64(want)).max() / max(np.abs(np.float64(want)).max(), 1e-30))


def read_tensors(path):
    """The tensors of a .l3m v1 file (src/model.h:28-57): name -> (dtype, shape, bytes as uint8 [rows, row_bytes])
    for matrices, (dtype, shape, bytes) otherwise, and the header's dims."""
    import struct
    raw = np.fromfile(path, np.uint8)
    dims = struct.unpack_from("<7I", raw, 28)
    n_tensors, = struct.unpack_from("<I", raw, 64)
    toc, = struct.unpack_from("<Q", raw, 72)
    out = {}
    for i in range(n_tensors):
        e = toc + 120 * i
        name = bytes(raw[e:e + 64]).split(b"\0")[0].decode()
        dtype, ndim = struct.unpack_from("<2I", raw, e + 64)
        shape = struct.unpack_from("<4Q", raw, e + 72)[:ndim]
        off, nbytes = struct.unpack_from("<2Q", raw, e + 104)
        data = raw[off:off + nbytes]
        if ndim == 2:
            data = data.reshape(shape[0], -1)
        out[name] = (dtype, shape, data)
    return out, dict(zip(("dim", "n_layers", "n_heads", "n_kv_heads", "ffn_dim", "vocab", "ctx"), dims))
