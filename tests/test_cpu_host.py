"""CPU checks of the host side of the GPU backend (no GPU needed): the C ABI is complete and fails loudly
without a device, the .l3m reader enforces the reference reader's rules, the lane-tile packing that the
kernels read matches the file blocks and the reference's own tile layout, and the seeded generator is
deterministic and shaped as specified.
"""
import ctypes as C
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import l3m_amd as A
from conftest import ROOT
from weights import BF16, F32, MXFP4, Q4_0, Q8_0, extremes, rows

HEADER = ROOT / "include" / "l3m_hip.h"
NO_GPU = not os.path.exists("/dev/kfd")


def header_functions():
    text = re.sub(r"//[^\n]*", "", HEADER.read_text())
    names = set(re.findall(r"\b(l3m_[a-z0-9_]+)\s*\(", text))
    names |= set(re.findall(r"extern const \w+ (l3m_\w+);", text))
    return sorted(n for n in names if not n.endswith("_fn"))


# ------------------------------------------------------------------------------------------ ABI

def test_every_declared_symbol_is_exported():
    lib = C.CDLL(str(ROOT / "l3m_amd" / "libl3m_hip.so"))
    names = header_functions()
    assert len(names) > 50
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in include/l3m_hip.h but not exported: {missing}"


def test_python_binding_covers_the_header():
    """Every function of the header that takes no FILE* has a ctypes signature in l3m_amd._SIG."""
    skip = {"l3m_print_hw", "l3m_chatml", "l3m_kernels_hip"}
    missing = [n for n in header_functions() if n not in A._SIG and n not in skip]
    assert not missing


def split_args(args):
    """A C parameter list split at its top-level commas (a function-pointer parameter stays whole)."""
    out, depth, cur = [], 0, ""
    for ch in args:
        depth += ch == "("
        depth -= ch == ")"
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip() not in ("", "void"):
        out.append(cur.strip())
    return out


def test_python_signatures_match_the_header():
    """Each ctypes signature has the header's number of parameters, pointers where the header has
    pointers and scalars where it has scalars (a missing parameter would turn a device pointer into a
    32-bit int on the call)."""
    text = re.sub(r"/\*.*?\*/", "", re.sub(r"//[^\n]*", "", HEADER.read_text()), flags=re.S)
    decls = re.findall(r"\b(l3m_\w+)\s*\(((?:[^;{()]|\([^()]*\))*)\)\s*;", text)
    checked, bad = 0, []
    for name, args in decls:
        if name not in A._SIG:
            continue
        params, (_, codes) = split_args(args), A._SIG[name]
        kinds = ["p" if "*" in a or "(" in a else "s" for a in params]
        want = ["s" if c in (C.c_int, C.c_int32, C.c_uint16, C.c_uint64, C.c_longlong, C.c_size_t, C.c_float, C.c_double) else "p"
            for c in codes]
        checked += 1
        if kinds != want:
            bad.append((name, params, want))
    assert checked > 50 and not bad, bad


def test_model_api_matches_the_reference_struct_layouts():
    """l3m_opts and l3m_perf have the reference's field order and sizes (src/l3m.h:10-29)."""
    assert [f[0] for f in A.Opts._fields_] == ["cpus", "n_cpus", "ctx", "reference", "force", "verbose", "cold"]
    assert [f[0] for f in A.Perf._fields_] == ["tokens", "ns_token", "ns_compute", "ns_wait", "bytes_token", "l2_bytes",
                                               "l3_miss", "dram_bytes", "energy_j", "llc_occupancy"]
    assert C.sizeof(A.Opts) == 32 and C.sizeof(A.Perf) == 80


@pytest.mark.skipif(not NO_GPU, reason="checks the behaviour on a host without a GPU")
def test_no_gpu_means_no_table_and_no_model(tmp_path):
    code = f"""
import sys, ctypes as C
sys.path.insert(0, {str(ROOT)!r})
import l3m_amd as A
lib = A.lib()
assert lib.l3m_hip_kernels_usable() == 0
assert C.c_char.in_dll(lib, "l3m_kernels_hip")                  # the table is there; the GPU is not
assert not hasattr(lib, "l3m_kernels_pick") and not hasattr(lib, "l3m_kernels_usable")   # dispatch.c's names
p = A.write_model({str(tmp_path / 'm.l3m')!r}, A.Config("t", 64, 1, 2, 2, 96, 300, 32, "q8_0"))
assert not lib.l3m_load(str(p).encode(), None)
print("no-gpu ok")
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "no-gpu ok" in r.stdout
    assert "no usable HIP device" in r.stderr


@pytest.mark.skipif(not NO_GPU, reason="checks the behaviour on a host without a GPU")
def test_reference_dispatcher_falls_back_without_gpu():
    """The reference's own dispatcher, built with the "hip" table (oracle/_ref/libl3m_ref_hip.so): without a
    GPU, L3M_ISA=hip is refused with the reference's message and its best CPU table is picked
    (dispatch.c:28-36), and l3m_kernels_usable(&l3m_kernels_hip) is 0."""
    from oracle.oracle import Reference
    if not Reference.available(Reference.HIP_PATH):
        pytest.skip("oracle/_ref/libl3m_ref_hip.so was not built (no reference sources)")
    code = f"""
import sys, ctypes as C
sys.path.insert(0, {str(ROOT)!r})
from oracle.oracle import Reference, _Table
plain = Reference()
best, _ = plain.pick()                               # L3M_ISA unset in that library's call
import os
os.environ["L3M_ISA"] = "hip"
r = Reference(Reference.HIP_PATH)
name, addr = r.pick()
hip = _Table.in_dll(r.lib, "l3m_kernels_hip")
print("picked", name, "best", best, "usable", r.lib.l3m_kernels_usable(C.addressof(hip)))
"""
    env = dict(os.environ)
    env.pop("L3M_ISA", None)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    _, picked, _, best, _, usable = r.stdout.split()
    assert picked == best and best in ("avx512", "avx2") and usable == "0", r.stdout
    assert f"l3m: L3M_ISA=hip not available here, using {best}" in r.stderr, r.stderr


@pytest.mark.parametrize("dtype", [Q4_0, MXFP4], ids=["q4_0", "mxfp4"])
def test_widened_rows_dequantize_bit_exact(oracle, dtype):
    """The q8_0 rows a q4_0 (or f16-scaled mxfp4) body's step matrices are stored as (l3m_widen_rows, the
    host conversion of the upload) hold exactly the file blocks' values (pack.c:55-62), zero rows stay zero,
    and an mxfp4 block whose scale 2^(e-128) is no f16 is refused unless its codes are all zero."""
    lib = A.lib()
    n, k = 24, 1376
    w = rows(dtype, n, k, seed=11 + dtype)
    if dtype == MXFP4:
        for i in range(n):                           # the f16 range of 2^(e - 128): 104 <= e <= 143
            w[i, 0::17] = 104 + (i * 7 + np.arange(k // 32)) % 40
    src = [w[i] if i < n - 2 else None for i in range(n)]
    ptrs = (C.c_void_p * n)(*[None if r is None else r.ctypes.data for r in src])
    out = np.zeros((n, k // 32 * 34), np.uint8)
    assert lib.l3m_widen_rows(dtype, n, k, ptrs, out.ctypes.data) == 0
    want = oracle.dequant(dtype, w[:n - 2], k)
    got = oracle.dequant(Q8_0, out[:n - 2], k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not out[n - 2:].any()                     # NULL rows: zero blocks, as the step's padding rows
    if dtype == MXFP4:
        bad = w[:1].copy()
        bad[0, 0] = 200                              # 2^72: no f16
        p1 = (C.c_void_p * 1)(bad.ctypes.data)
        assert lib.l3m_widen_rows(dtype, 1, k, p1, out.ctypes.data) == -1
        bad[0, 1:17] = 0                             # ... unless the block's codes are all zero
        assert lib.l3m_widen_rows(dtype, 1, k, p1, out.ctypes.data) == 0


def test_parse_cpus():
    lib = A.lib()
    buf = (C.c_int * 16)()
    assert lib.l3m_parse_cpus(b"0-3,8,10-11", buf, 16) == 7 and list(buf[:7]) == [0, 1, 2, 3, 8, 10, 11]
    for bad in (b"", b"3-1", b"1,", b"a", b"1-", b"-2"):
        assert lib.l3m_parse_cpus(bad, buf, 16) == -1, bad
    assert lib.l3m_parse_cpus(b"0-31", buf, 16) == -1


# ------------------------------------------------------------------------------------- the reader

def load_stderr(path):
    """l3m_load in a child process: its return and what it printed (the file is checked before the GPU)."""
    code = f"import sys; sys.path.insert(0, {str(ROOT)!r}); import l3m_amd as A; print(bool(A.lib().l3m_load({str(path)!r}.encode(), None)))"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    return r.stdout.strip(), r.stderr


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    return A.write_model(tmp_path_factory.mktemp("reader") / "tiny.l3m", A.Config("t", 64, 2, 2, 1, 96, 300, 32, "q4_0"))


def corrupt(src, dst, offset, data):
    b = bytearray(src.read_bytes())
    b[offset:offset + len(data)] = data
    dst.write_bytes(bytes(b))
    return dst


def toc_entry(path, name):
    b = path.read_bytes()
    n = int.from_bytes(b[64:68], "little")
    toc = int.from_bytes(b[72:80], "little")
    for i in range(n):
        e = toc + i * 120
        if b[e:e + 64].rstrip(b"\0").decode() == name:
            return e
    raise KeyError(name)


@pytest.mark.parametrize("what,patch,message", [
    ("magic", lambda p: (0, b"xyz"), "not an l3m v1 file"),
    ("version", lambda p: (4, (2).to_bytes(4, "little")), "not an l3m v1 file"),
    ("toc past the end", lambda p: (72, (1 << 40).to_bytes(8, "little")), "truncated file"),
    ("head_dim", lambda p: (36, (3).to_bytes(4, "little")), "bad config"),
    ("dtype", lambda p: (toc_entry(p, "blk.0.wq") + 64, (9).to_bytes(4, "little")), "unknown dtype"),
    ("nbytes", lambda p: (toc_entry(p, "blk.0.wq") + 112, (7).to_bytes(8, "little")), "do not match its shape"),
    ("offset", lambda p: (toc_entry(p, "blk.0.wq") + 104, (65).to_bytes(8, "little")), "misaligned or outside"),
    # [64, 96] -> [96, 64] keeps the byte count of a q4_0 matrix: the entry is sound, the model shape is not
    ("shape", lambda p: (toc_entry(p, "blk.1.w_down") + 72, (96).to_bytes(8, "little") + (64).to_bytes(8, "little")),
     "tensor blk.1.w_down: expected [64, 96]"),
    ("missing", lambda p: (toc_entry(p, "norm"), b"nrm\0"), "tensor norm missing"),
    ("qkv dtypes", lambda p: (toc_entry(p, "blk.0.wk") + 64, (2).to_bytes(4, "little")), None),
])
def test_reader_rejects(tmp_path, tiny_file, what, patch, message):
    off, data = patch(tiny_file)
    bad = corrupt(tiny_file, tmp_path / "bad.l3m", off, data)
    ok, err = load_stderr(bad)
    assert ok == "False"
    assert "no usable HIP device" not in err, "the file must be rejected before the device is looked for"
    if message:
        assert message in err, err
    assert err.startswith(f"l3m: {bad}:")


def test_reader_accepts_good_file(tiny_file):
    ok, err = load_stderr(tiny_file)
    if NO_GPU:
        assert ok == "False" and "no usable HIP device" in err and str(tiny_file) not in err


def test_truncated_file_is_rejected(tmp_path, tiny_file):
    p = tmp_path / "short.l3m"
    p.write_bytes(tiny_file.read_bytes()[:-100])
    ok, err = load_stderr(p)
    assert ok == "False" and str(p) in err


# --------------------------------------------------------------------------------- lane-tile layout

def lt_decode(dtype, q, s, n, k, oracle):
    """Rows back from the lane-tile planes: [tile][block][16 rows][QBYTES] + [tile][block][16][SBYTES]."""
    qb, sb = A.lib().l3m_lt_qbytes(dtype), A.lib().l3m_lt_sbytes(dtype)
    nb, tiles = (k + 31) // 32, (n + 15) // 16
    qv = q.reshape(tiles, nb, 16, qb)
    sv = s.reshape(tiles, nb, 16, sb) if sb else None
    out = np.zeros((n, nb * 32), np.float32)
    for r in range(n):
        t, c = divmod(r, 16)
        for b in range(nb):
            if sb:
                block = np.concatenate([sv[t, b, c], qv[t, b, c]])
                out[r, b * 32:(b + 1) * 32] = oracle.dequant(dtype, block[None, :], 32)[0]
            else:
                out[r, b * 32:(b + 1) * 32] = oracle.dequant(dtype, qv[t, b, c][None, :], 32)[0]
    return out[:, :k]


@pytest.mark.parametrize("dtype", [F32, BF16, Q8_0, Q4_0, MXFP4])
@pytest.mark.parametrize("n,k", [(16, 64), (37, 96), (5, 288)])
def test_lane_tiles_hold_the_file_blocks(oracle, dev_free, dtype, n, k):
    r = extremes(dtype, rows(dtype, n, k, seed=n + k), k)
    q, s = dev_free.pack_rows(dtype, r, k)
    assert len(q) == A.lib().l3m_lt_quant_size(dtype, n, k) and len(s) == A.lib().l3m_lt_scale_size(dtype, n, k)
    np.testing.assert_array_equal(lt_decode(dtype, q, s, n, k, oracle), oracle.dequant(dtype, r, k))


@pytest.mark.parametrize("dtype", [F32, BF16, Q8_0, Q4_0, MXFP4])
def test_lane_tiles_from_reference_tiles(reference, dev_free, dtype):
    """The kernel table's repacking of the reference's 16-row tiles (kernels.h:1-11) equals packing the
    file rows directly."""
    n, k = 40, 128
    r = extremes(dtype, rows(dtype, n, k, seed=9), k)
    tiles = reference.pack_tiles(dtype, list(r) + [None] * (-n % 16), k)
    nt = (n + 15) // 16
    qs, ss = A.lib().l3m_lt_quant_size(dtype, nt * 16, k), A.lib().l3m_lt_scale_size(dtype, nt * 16, k)
    q2, s2 = np.zeros(qs, np.uint8), np.zeros(max(ss, 1), np.uint8)
    A.lib().l3m_lt_pack_ltiles(dtype, nt, k, tiles.ctypes.data, q2.ctypes.data, s2.ctypes.data)
    q1, s1 = dev_free.pack_rows(dtype, list(r) + [None] * (-n % 16), k)
    np.testing.assert_array_equal(s2[:ss], s1)
    # rows past n: the reference pads q8_0 tiles with raw zero bytes (code -128 beside a zero scale), so
    # only the real rows' quant bytes are compared
    qb, nb = A.lib().l3m_lt_qbytes(dtype), (k + 31) // 32
    real = (np.arange(nt * 16) < n).reshape(nt, 1, 16, 1)
    q1v, q2v = q1.reshape(nt, nb, 16, qb), q2.reshape(nt, nb, 16, qb)
    np.testing.assert_array_equal(np.where(real, q2v, 0), np.where(real, q1v, 0))


# ----------------------------------------------------------------------------------- generator

def test_generator_normal_moments():
    lib = A.lib()
    v = np.array([lib.l3m_gen_normal(12345, i) for i in range(1 << 16)], np.float64)
    assert abs(v.mean()) < 0.02 and abs(v.std() - 1) < 0.02
    assert np.abs(v).max() <= 2 * np.sqrt(3) + 1e-6            # Irwin-Hall of four: bounded at 2*sqrt(3)
    w = np.array([lib.l3m_gen_normal(12345, i) for i in range(64)], np.float64)
    np.testing.assert_array_equal(w, v[:64])                  # counter-based: same stream, same values


def test_prompt_ids_in_range_and_seeded():
    a, b = A.prompt(1, 32000, 64), A.prompt(2, 32000, 64)
    assert a == A.prompt(1, 32000, 64) and a != b
    assert all(0 <= t < 32000 for t in a + b)


def test_model_files_are_deterministic(tmp_path):
    cfg = A.Config("t", 64, 1, 2, 2, 96, 300, 32, "mxfp4")
    p1, p2 = A.write_model(tmp_path / "a.l3m", cfg, seed=3), A.write_model(tmp_path / "b.l3m", cfg, seed=3)
    p3 = A.write_model(tmp_path / "c.l3m", cfg, seed=4)
    assert p1.read_bytes() == p2.read_bytes() != p3.read_bytes()
