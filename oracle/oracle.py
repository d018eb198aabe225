"""TEST INFRASTRUCTURE ONLY: ctypes access to the checker.

`Oracle` wraps liboracle.so, the scalar C restatement of fpedd/l3m's decode path (oracle.c).
`Reference` wraps _ref/libl3m_ref.so, the reference compiled from its own sources (Makefile here); it is
present where /root/reference was when the checker was built, and absent otherwise.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
"""
import ctypes as C
import os
from pathlib import Path

import numpy as np

import l3m_amd
from l3m_amd import TOKEN_CALLBACK, Opts, Perf

HERE = Path(__file__).resolve().parent
F32, BF16, Q8_0, Q4_0, MXFP4 = range(5)

_f = C.POINTER(C.c_float)
_i8 = C.POINTER(C.c_int8)
_i32 = C.POINTER(C.c_int32)
_u16 = C.POINTER(C.c_uint16)


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


class Oracle:
    def __init__(self, path=HERE / "liboracle.so"):
        if not Path(path).exists():
            raise OSError(f"{path} missing: build it with `make -C oracle`")
        lib = self.lib = C.CDLL(str(path))
        sig = {
            "or_f16_f32": (C.c_float, [C.c_uint16]),
            "or_bf16_f32": (C.c_float, [C.c_uint16]),
            "or_f32_bf16": (C.c_uint16, [C.c_float]),
            "or_row_bytes": (C.c_size_t, [C.c_int, C.c_int]),
            "or_dequant_row": (None, [_f, C.c_int, C.c_void_p, C.c_int]),
            "or_vec_prepare": (None, [C.c_int, _f, C.c_int, _u16, _i8, _f, _i32]),
            "or_gemv": (None, [C.c_int, _f, C.c_void_p, C.c_int, C.c_int, _f]),
            "or_gemv_prepared": (None, [C.c_int, _f, C.c_void_p, C.c_int, C.c_int, _f, _u16, _i8, _f, _i32]),
            "or_rmsnorm": (None, [_f, _f, _f, C.c_int, C.c_float]),
            "or_rope": (None, [_f, C.c_int, C.c_int, C.c_int, C.c_float]),
            "or_silu_mul": (None, [_f, _f, C.c_int]),
            "or_attend": (None, [_f, _f, _u16, _u16, C.c_int, C.c_int, C.c_int]),
            "or_load": (C.c_void_p, [C.c_char_p, C.c_int, C.c_int]),
            "or_free": (None, [C.c_void_p]),
            "or_vocab": (C.c_int, [C.c_void_p]),
            "or_ctx": (C.c_int, [C.c_void_p]),
            "or_logits": (_f, [C.c_void_p]),
            "or_forward": (None, [C.c_void_p, C.c_int32, C.c_int, C.c_int]),
            "or_generate": (C.c_int, [C.c_void_p, _i32, C.c_int, C.c_int, _i32]),
            "or_rand01": (C.c_double, [C.POINTER(C.c_uint64)]),
            "or_seed_state": (C.c_uint64, [C.c_uint64]),
            "or_sample": (C.c_int, [_f, C.c_int, C.c_float, C.POINTER(C.c_uint64)]),
            "or_generate_sampled": (C.c_int, [C.c_void_p, _i32, C.c_int, C.c_int, C.c_float, C.c_uint64, _i32]),
            "or_kv_rows": (None, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, _u16, _u16]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args

    # --- blocks and kernels
    def row_bytes(self, dtype, k):
        return self.lib.or_row_bytes(dtype, k)

    def dequant(self, dtype, rows, k):
        """rows: uint8 [n, row_bytes] -> float32 [n, k]."""
        rows = np.ascontiguousarray(rows, dtype=np.uint8).reshape(-1, self.row_bytes(dtype, k))
        out = np.zeros((len(rows), k), np.float32)
        for i, r in enumerate(rows):
            self.lib.or_dequant_row(_p(out[i], _f), dtype, r.ctypes.data, k)
        return out

    def prepare(self, dtype, x):
        x = np.ascontiguousarray(x, np.float32)
        n = len(x)
        bf, q8 = np.zeros(n, np.uint16), np.zeros(n, np.int8)
        scale, s = np.zeros(max(n // 32, 1), np.float32), np.zeros(max(n // 32, 1), np.int32)
        self.lib.or_vec_prepare(dtype, _p(x, _f), n, _p(bf, _u16), _p(q8, _i8), _p(scale, _f), _p(s, _i32))
        return {"bf16": bf, "q8": q8, "scale": scale[: n // 32], "sum": s[: n // 32]}

    def gemv(self, dtype, rows, nrows, k, x):
        rows = np.ascontiguousarray(rows, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(nrows, np.float32)
        self.lib.or_gemv(dtype, _p(y, _f), rows.ctypes.data, nrows, k, _p(x, _f))
        return y

    def rmsnorm(self, x, w, eps):
        x, w = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32)
        y = np.zeros_like(x)
        self.lib.or_rmsnorm(_p(y, _f), _p(x, _f), _p(w, _f), len(x), eps)
        return y

    def rope(self, v, n_heads, hd, pos, theta):
        v = np.array(v, np.float32)
        self.lib.or_rope(_p(v, _f), n_heads, hd, pos, theta)
        return v

    def silu_mul(self, h, g):
        h, g = np.array(h, np.float32), np.ascontiguousarray(g, np.float32)
        self.lib.or_silu_mul(_p(h, _f), _p(g, _f), len(h))
        return h

    def attend(self, q, k, v, pos, hd, stride):
        q = np.ascontiguousarray(q, np.float32)
        k, v = np.ascontiguousarray(k, np.uint16), np.ascontiguousarray(v, np.uint16)
        out = np.zeros(hd, np.float32)
        self.lib.or_attend(_p(out, _f), _p(q, _f), _p(k, _u16), _p(v, _u16), pos, hd, stride)
        return out

    # --- temperature sampling (engine.c:98-101, 284-287, 364-379, 555)
    def seed_state(self, seed):
        return self.lib.or_seed_state(seed % (1 << 64))

    def rand01(self, state):
        """(the draw, the next state) of xorshift64* from state."""
        st = C.c_uint64(state)
        u = self.lib.or_rand01(C.byref(st))
        return u, st.value

    def sample(self, logits, temp, state):
        """(the token, the next state): the reference path's pick from logits at temperature temp."""
        x = np.ascontiguousarray(logits, np.float32)
        st = C.c_uint64(state)
        tok = self.lib.or_sample(_p(x, _f), len(x), temp, C.byref(st))
        return tok, st.value

    # --- model
    def load(self, path, ctx=0, ref=False):
        h = self.lib.or_load(os.fsencode(str(path)), ctx, int(ref))
        if not h:
            raise OSError(f"oracle could not read {path}")
        return OracleModel(self, h)


class OracleModel:
    def __init__(self, o, h):
        self.o, self.h = o, h
        self.vocab, self.ctx = o.lib.or_vocab(h), o.lib.or_ctx(h)

    def __del__(self):
        if getattr(self, "h", None):
            self.o.lib.or_free(self.h)
            self.h = None

    def generate(self, prompt, max_new, temperature=0.0, seed=0):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(max_new, 1), np.int32)
        if temperature > 0:
            n = self.o.lib.or_generate_sampled(self.h, _p(p, _i32), len(p), max_new, temperature, seed % (1 << 64), _p(out, _i32))
        else:
            n = self.o.lib.or_generate(self.h, _p(p, _i32), len(p), max_new, _p(out, _i32))
        return out[:n].tolist()

    def logits(self):
        return np.ctypeslib.as_array(self.o.lib.or_logits(self.h), shape=(self.vocab,)).copy()

    def forward(self, tok, pos, logits=True):
        """One position (engine.c:230-281): the logits after it when asked for (teacher forcing)."""
        self.o.lib.or_forward(self.h, tok, pos, int(logits))
        return self.logits() if logits else None

    def kv_rows(self, layer, kvh, pos0, n, hd):
        """bf16 K and V rows [pos0, pos0 + n) of kv head kvh in layer `layer`, uint16 [n, hd] each."""
        k, v = np.zeros((n, hd), np.uint16), np.zeros((n, hd), np.uint16)
        self.o.lib.or_kv_rows(self.h, layer, kvh, pos0, n, _p(k, _u16), _p(v, _u16))
        return k, v


class _Vec(C.Structure):
    _fields_ = [("f32", _f), ("bf16", _u16), ("q8", _i8), ("scale", _f), ("sum", _i32)]


_GEMV = C.CFUNCTYPE(None, _f, C.c_void_p, C.c_int, C.c_int, C.POINTER(_Vec))
_ATTEND = C.CFUNCTYPE(None, _f, _f, _u16, _u16, C.c_int, C.c_int, C.c_int)


class _Table(C.Structure):
    _fields_ = [("name", C.c_char_p), ("gemv", _GEMV * 5), ("attend", _ATTEND)]


class Reference:
    """fpedd/l3m built from source (oracle/_ref): its kernel tables and its l3m.h engine."""
    PATH = HERE / "_ref" / "libl3m_ref.so"
    # the same library with its dispatcher able to pick l3m_kernels_hip (L3M_ISA=hip), linked against
    # libl3m_hip.so (the Makefile's _ref/libl3m_ref_hip.so)
    HIP_PATH = HERE / "_ref" / "libl3m_ref_hip.so"

    @classmethod
    def available(cls, path=None):
        return (path or cls.PATH).exists()

    def __init__(self, path=None):
        path = path or self.PATH
        if not path.exists():
            raise OSError(f"{path} missing: build it with `make -C oracle ref` where /root/reference exists")
        lib = self.lib = C.CDLL(str(path))
        # the reference's l3m.h entry points share the product's ctypes structs (same ABI); the rest are its
        # internal packing and prep functions (pack.c) and the kernel tables (kernels.h)
        api = {name: l3m_amd._SIG[name] for name in ("l3m_load", "l3m_free", "l3m_generate", "l3m_logits", "l3m_vocab",
                                                      "l3m_describe", "l3m_perf_read")}
        api["l3m_kernels_usable"] = (C.c_int, [C.c_void_p])           # dispatch.c:23
        api["l3m_encode"] = l3m_amd._SIG["l3m_encode"]
        api["l3m_kernels_pick"] = (C.c_void_p, [])                    # dispatch.c:28
        internal = {
            "l3m_tile_bytes": (C.c_size_t, [C.c_int, C.c_int]),
            "l3m_row_bytes": (C.c_size_t, [C.c_int, C.c_int]),
            "l3m_pack_tile": (None, [C.c_void_p, C.c_int, C.POINTER(C.c_void_p), C.c_int]),
            "l3m_vec_prepare": (None, [C.POINTER(_Vec), C.c_int, _f, C.c_int, C.c_void_p]),
            "l3m_dequant_row": (None, [_f, C.c_int, C.c_void_p, C.c_int]),
        }
        for name, (restype, argtypes) in {**api, **internal}.items():
            entry = getattr(lib, name)
            entry.restype, entry.argtypes = restype, argtypes
        self.tables = {n: _Table.in_dll(lib, f"l3m_kernels_{n}") for n in ("scalar", "avx2", "avx512")}

    def usable(self, name):
        return bool(self.lib.l3m_kernels_usable(C.addressof(self.tables[name])))

    def pick(self):
        """The dispatcher's choice (dispatch.c:28-36, L3M_ISA read at the call): the table's name and address."""
        p = self.lib.l3m_kernels_pick()
        return _Table.from_address(p).name.decode(), p

    def pack_tiles(self, dtype, rows, k):
        """File rows uint8 [n, row_bytes] (n a multiple of 16, None rows allowed as zeros) -> tile bytes."""
        n = len(rows)
        tb = self.lib.l3m_tile_bytes(dtype, k)
        out = np.zeros((n + 15) // 16 * tb, np.uint8)
        keep = [None if r is None else np.ascontiguousarray(r, np.uint8) for r in rows]
        for t in range((n + 15) // 16):
            ptrs = (C.c_void_p * 16)(*[(keep[t * 16 + c].ctypes.data if t * 16 + c < n and keep[t * 16 + c] is not None
                                        else None) for c in range(16)])
            self.lib.l3m_pack_tile(out[t * tb:].ctypes.data, dtype, ptrs, k)
        return out

    def prepare(self, dtype, x):
        x = np.ascontiguousarray(x, np.float32)
        scratch = np.zeros(2 * len(x) + 64, np.uint8)
        v = _Vec()
        self.lib.l3m_vec_prepare(C.byref(v), dtype, _p(x, _f), len(x), scratch.ctypes.data)
        return v, (x, scratch)

    def gemv(self, table, dtype, tiles, ntiles, k, x):
        v, keep = self.prepare(dtype, x)
        y = np.zeros(ntiles * 16, np.float32)
        self.tables[table].gemv[dtype](_p(y, _f), tiles.ctypes.data, ntiles, k, C.byref(v))
        return y

    def dequant(self, dtype, row, k):
        out = np.zeros(k, np.float32)
        self.lib.l3m_dequant_row(_p(out, _f), dtype, np.ascontiguousarray(row, np.uint8).ctypes.data, k)
        return out

    def attend(self, table, q, k, v, pos, hd, stride):
        out = np.zeros(hd, np.float32)
        q, k, v = (np.ascontiguousarray(a) for a in (q, k, v))
        self.tables[table].attend(_p(out, _f), _p(q, _f), _p(k, _u16), _p(v, _u16), pos, hd, stride)
        return out

    def load(self, path, ctx=0, reference=False, cpus=None):
        opts = Opts(ctx=ctx, reference=int(reference), force=1)
        if cpus:
            arr = (C.c_int * len(cpus))(*cpus)
            opts.cpus, opts.n_cpus = arr, len(cpus)
        h = self.lib.l3m_load(os.fsencode(str(path)), C.byref(opts))
        if not h:
            raise OSError(f"reference l3m_load failed for {path}")
        return RefModel(self, h)


class RefModel:
    def __init__(self, r, h):
        self.r, self.h = r, h
        self.vocab = r.lib.l3m_vocab(h)

    def __del__(self):
        if getattr(self, "h", None):
            self.r.lib.l3m_free(self.h)
            self.h = None

    def describe(self):
        return self.r.lib.l3m_describe(self.h).decode()

    def encode(self, text, add_bos=True, cap=None):
        raw = text.encode()
        cap = cap or len(raw) + 8
        out = (C.c_int32 * cap)()
        n = self.r.lib.l3m_encode(self.h, raw, int(add_bos), out, cap)
        return None if n < 0 else list(out[:n])

    def generate(self, prompt, max_new, temperature=0.0, seed=0):
        out = []
        cb = TOKEN_CALLBACK(lambda t, u: out.append(t) or 1)
        p = np.ascontiguousarray(prompt, np.int32)
        n = self.r.lib.l3m_generate(self.h, _p(p, _i32), len(p), max_new, temperature, seed % (1 << 64), cb, None)
        assert n == len(out)
        return out

    def logits(self):
        return np.ctypeslib.as_array(self.r.lib.l3m_logits(self.h), shape=(self.vocab,)).copy()

    def perf(self):
        p = Perf()
        if self.r.lib.l3m_perf_read(self.h, C.byref(p)):
            return None
        return {f: getattr(p, f) for f, _ in Perf._fields_}
