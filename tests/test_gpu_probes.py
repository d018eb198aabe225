"""The residency and exchange probes (the GPU analogues of the reference's bench/residency.c and
bench/exchange.c) run, stay bounded and report physically sensible figures: a warm working set that fits
one XCD's L2 streams faster than one that spills past it, 256 workgroups outrun 32 on a set too large for
any cache, an exchange round among workgroups of one XCD costs under 20 us and a graph node under 50 us,
and each step of the latency probe takes between 1 and 5000 shader clocks, an LDS hand-over through a
barrier more than a lone barrier.
"""
import ctypes as C

import pytest

import l3m_amd as A

pytestmark = pytest.mark.gpu


def stream(per_wg, xcds, passes=4):
    v = C.c_double()
    assert A.lib().l3m_probe_stream(per_wg, xcds, 32, passes, C.byref(v)) == 0
    return v.value


def test_stream_probe():
    print("case stream", flush=True)
    small = stream(64 << 10, 1, 16)                   # 2 MiB on one XCD: its L2
    big = stream(8 << 20, 1, 1)                       # 256 MiB on one XCD
    assert 0 < big < small
    wide = stream(4 << 20, 8, 1)                      # 1 GiB over all XCDs
    assert wide > big


@pytest.mark.parametrize("same", [1, 0])
def test_exchange_probe(same):
    print(f"case exchange same={same}", flush=True)
    v = C.c_double()
    assert A.lib().l3m_probe_exchange(8, same, 768, 500, C.byref(v)) == 0
    assert 0 < v.value < 20.0


def test_graph_node_probe():
    v = C.c_double()
    assert A.lib().l3m_probe_graph_node(64, 5, C.byref(v)) == 0
    assert 0 < v.value < 50.0


def test_latency_probe():
    print("case latency", flush=True)
    lib, v = A.lib(), C.c_double()
    got = {}
    for which in range(7):
        assert lib.l3m_probe_latency(which, 1024, C.byref(v)) == 0
        got[which] = v.value
        assert 1.0 < v.value < 5000.0, (which, v.value)
    assert got[0] > got[4]                           # write + barrier + read + barrier > a barrier
    lib.l3m_dev_clear_error()
    assert lib.l3m_probe_latency(0, 96, C.byref(v)) != 0   # threads not a power of two: refused
    assert b"probe_latency" in lib.l3m_dev_error()
    lib.l3m_dev_clear_error()
