"""The allocation-free attention entry point (l3m_hip_attend_noalloc, no counterpart in the reference)
against the kernel table's attend (l3m_kernels_hip.attend), through the C ABI: bit-identical outputs on
two calls in a row, the second with a smaller input (the static array keeps the first call's contents), and
a clear refusal of a call past the array's size."""
import ctypes as C

import numpy as np
import pytest

import l3m_amd as A

pytestmark = pytest.mark.gpu
_f, _u16 = C.POINTER(C.c_float), C.POINTER(C.c_uint16)


def inputs(seed, pos, hd, stride):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal(hd) * 3).astype(np.float32)
    k = rng.integers(0, 1 << 16, pos * stride + hd, dtype=np.uint16) & 0xBF7F
    v = rng.integers(0, 1 << 16, pos * stride + hd, dtype=np.uint16) & 0xBF7F
    return q, k.astype(np.uint16), v.astype(np.uint16)


def call(fn, q, k, v, pos, hd, stride):
    out = np.full(hd, np.nan, np.float32)
    rc = fn(out.ctypes.data_as(_f), q.ctypes.data_as(_f), k.ctypes.data_as(_u16), v.ctypes.data_as(_u16), pos, hd, stride)
    return rc, out


def test_noalloc_attend_matches_table_attend():
    from oracle.oracle import _Table
    lib = A.lib()
    table = _Table.in_dll(lib, "l3m_kernels_hip")
    noalloc = lambda *a: lib.l3m_hip_attend_noalloc(*[C.cast(x, C.c_void_p) if isinstance(x, C._Pointer) else x for x in a])
    table_attend = lambda *a: (table.attend(*a), 0)[1]
    for seed, (pos, hd, stride) in enumerate([(3000, 64, 192), (40, 48, 96)]):   # the second call is smaller
        print(f"noalloc attend: pos {pos} hd {hd} stride {stride}", flush=True)
        q, k, v = inputs(seed, pos, hd, stride)
        rc, got = call(noalloc, q, k, v, pos, hd, stride)
        assert rc == 0
        _, want = call(table_attend, q, k, v, pos, hd, stride)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # past the array: refused on the host, nothing launched, the next call still works
    pos, hd, stride = 9000, 64, 128
    q, k, v = inputs(7, pos, hd, stride)
    rc, _ = call(noalloc, q, k, v, pos, hd, stride)
    assert rc == -1 and b"staging array" in lib.l3m_dev_error()
    lib.l3m_dev_clear_error()
    q, k, v = inputs(8, 5, 32, 32)
    rc, got = call(noalloc, q, k, v, 5, 32, 32)
    _, want = call(table_attend, q, k, v, 5, 32, 32)
    assert rc == 0 and np.array_equal(got.view(np.uint32), want.view(np.uint32))
