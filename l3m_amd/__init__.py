"""l3m-mi355x: ctypes access to libl3m_hip.so, the gfx950 backend of l3m's batch-1 decode path.

`Model` mirrors the reference's Python wrapper (python/l3m/__init__.py:53-157) over the same l3m.h API;
the reference wrapper itself also works with L3M_LIB pointing at libl3m_hip.so. `Device` exposes the
device-level kernels (include/l3m_hip.h, part 3) for tests and benchmarks. `write_model` writes the
seeded synthetic models of the benchmark configurations.

There is no CPU fallback: if the library is missing this module raises, and without a GPU `Model` raises.
"""
import atexit
import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libl3m_hip.so"
F32, BF16, Q8_0, Q4_0, MXFP4 = range(5)
DTYPES = {"f32": F32, "bf16": BF16, "q8_0": Q8_0, "q4_0": Q4_0, "mxfp4": MXFP4}
DTYPE_NAMES = {v: k for k, v in DTYPES.items()}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, MXFP4: 17}

TOKEN_CALLBACK = C.CFUNCTYPE(C.c_int, C.c_int32, C.c_void_p)
_f = C.POINTER(C.c_float)
_i32 = C.POINTER(C.c_int32)
_u16 = C.POINTER(C.c_uint16)


def _struct(name, fields):
    return type(name, (C.Structure,), {"_fields_": fields})


# The C structs of include/l3m_hip.h, field for field (l3m_opts and l3m_perf have the layout of src/l3m.h).
Opts = _struct("Opts", [("cpus", C.POINTER(C.c_int))] + [(n, C.c_int) for n in "n_cpus ctx reference force verbose cold".split()])
PERF_FIELDS = "tokens ns_token ns_compute ns_wait bytes_token l2_bytes l3_miss dram_bytes energy_j llc_occupancy".split()
Perf = _struct("Perf", [(n, C.c_double) for n in PERF_FIELDS])
DMat = _struct("DMat", [("q", C.c_void_p), ("s", C.c_void_p)] + [(n, C.c_int) for n in "rows tiles nb dtype".split()])
GenSpec = _struct("GenSpec", [("arch", C.c_char_p)] + [(n, C.c_int) for n in "dim n_layers n_heads n_kv_heads ffn_dim vocab ctx".split()]
                  + [("rope_theta", C.c_float), ("norm_eps", C.c_float)] + [(n, C.c_int) for n in "dtype head_dtype tied".split()]
                  + [("seed", C.c_uint64), ("std", C.c_float), ("norm_jitter", C.c_float), ("bos", C.c_int), ("eos", C.c_int)])

# Signature table: one line per exported function, "name result arg...", in the type codes below.
_CODES = {"v": None, "i": C.c_int, "I": C.c_int32, "w": C.c_uint16, "q": C.c_uint64, "l": C.c_longlong, "z": C.c_size_t, "f": C.c_float,
          "d": C.c_double, "p": C.c_void_p, "s": C.c_char_p, "*i": C.POINTER(C.c_int), "*I": _i32, "*f": _f,
          "*d": C.POINTER(C.c_double),
          "**": C.POINTER(C.c_void_p), "O": C.POINTER(Opts), "P": C.POINTER(Perf), "M": C.POINTER(DMat),
          "G": C.POINTER(GenSpec), "cb": TOKEN_CALLBACK}
_SIGNATURES = """
l3m_load p s O                  | l3m_free v p                   | l3m_logits *f p
l3m_generate i p *I i i f q cb p | l3m_vocab i p                 | l3m_ctx i p
l3m_describe s p                | l3m_encode i p s i *I i        | l3m_decode p p I *i
l3m_bos i p                     | l3m_eos i p                    | l3m_perf_read i p P
l3m_parse_cpus i s *i i         | l3m_hip_kernels_usable i
l3m_hip_last_error s            | l3m_dev_init i                 | l3m_dev_error s
l3m_dev_clear_error v           | l3m_dev_name s                 | l3m_dev_alloc p z
l3m_dev_free v p                | l3m_dev_upload i p p z         | l3m_dev_download i p p z
l3m_dev_sync i                  | l3m_dev_stream p               | l3m_lt_qbytes i i
l3m_dev_copy i p p z p          | l3m_dev_shutdown v
l3m_lt_sbytes i i               | l3m_lt_quant_size z i i i      | l3m_lt_scale_size z i i i
l3m_lt_pack_rows v i i i ** p p | l3m_lt_pack_ltiles v i i i p p p | l3m_act_bytes z i i
l3m_k_prep i i p i p p          | l3m_k_gemv i M p i p p         | l3m_k_attend i p p p p i i i p
l3m_k_rmsnorm i p p p i f p     | l3m_k_rope i p i i i p p       | l3m_k_silu_mul i p p i p
l3m_k_argmax i p i p p          | l3m_rope_table v *f i i f      | l3m_bench_decode d p *I i i
l3m_bench_kernel d p i i i i    | l3m_kernel_bytes d p i i       | l3m_weight_bytes d p
l3m_time_gemv d M i p i p i     | l3m_gen_write i G s            | l3m_gen_prompt v q i i *I
l3m_gen_u64 q q q               | l3m_gen_normal f q q           | l3m_quantize_row v i p *f i
l3m_f32_to_f16 w f               | l3m_decode_persistent i p      | l3m_decode_timer i i *d *i
l3m_decode_work v p *d          | l3m_logits_at i p i *f         | l3m_bench_decode_t d p *I i i f q
l3m_prefill_positions i p       | l3m_probe_stream i z i i i *d   | l3m_probe_exchange i i i i i *d
l3m_probe_graph_node i i i *d   | l3m_probe_latency i i i *d
l3m_k_dequant i M i i p p       | l3m_attention_mode i i i i i   | l3m_k_attend_decode i i p p p p i i i i i p
l3m_dev_evict i p z p           | l3m_decode_attention i p       | l3m_kv_rows i p i i i i p p
l3m_decode_window i p
l3m_k_step_mv i i i M p i p i p  | l3m_step_matvec i p i i i *f *f | l3m_step_layout v p *i
l3m_widen_rows i i i i ** p | l3m_decode_spin_limit v p l | l3m_time_launch_interval d i
l3m_tokenize i s s i *I i | l3m_head_dim i p | l3m_gemv_matrix_cores i i
l3m_time_read d ** i z i         | l3m_hip_attend_noalloc i p p p p i i i | l3m_phase_stamps i i i i p
"""
_SIG = {}
for _entry in _SIGNATURES.replace("\n", "|").split("|"):
    if _entry.strip():
        _name, _res, *_args = _entry.split()
        _SIG[_name] = (_CODES[_res], [_CODES[a] for a in _args])

_lib = None


def lib():
    """The backend library; raises if it was not built (no fallback exists)."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("L3M_HIP_LIB", LIB_PATH))
        if not path.exists():
            raise OSError(f"{path} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                          "or `make -C l3m_amd/csrc`")
        handle = C.CDLL(str(path))
        for name, (res, args) in _SIG.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
        # the library's stream and events go before the interpreter exits, while HIP (and a profiler
        # wrapping it) is still up
        atexit.register(handle.l3m_dev_shutdown)
    return _lib


def _p(a, t=C.c_void_p):
    return a.ctypes.data_as(t) if t is not C.c_void_p else C.c_void_p(a.ctypes.data)


# --------------------------------------------------------------------------------------- model API

class _TokenSink:
    """The on_token bridge of one generate call: records ids, asks the Python callback, and keeps an
    exception raised there to re-raise once the C call has returned."""

    def __init__(self, on_token):
        self.ids, self.on_token, self.error = [], on_token, None
        self.c_func = TOKEN_CALLBACK(self._called)

    def _called(self, tok, _user):
        self.ids.append(int(tok))
        if self.on_token is None:
            return 1
        try:
            keep = self.on_token(int(tok))
        except BaseException as exc:      # noqa: BLE001 - carried across the C frame
            self.error = exc
            return 0
        return 0 if keep is False else 1


class Model:
    """A .l3m file loaded on the GPU with a KV cache of ctx positions (0: min(model, 512)). The arguments
    are those of the reference's Python Model (python/l3m/__init__.py:53-68); cpus and force are accepted
    for compatibility and have no meaning on one GPU; cold evicts the caches before each forward pass."""
    _m = None

    def __init__(self, path, cpus=None, ctx=0, reference=False, force=False, verbose=False, cold=False):
        if ctx and ctx < 2:
            raise ValueError(f"ctx {ctx} leaves no room after a one-token prompt")
        self._lib = lib()
        opts = Opts()
        opts.ctx, opts.reference, opts.force, opts.verbose, opts.cold = ctx, int(reference), int(force), int(verbose), int(cold)
        handle = self._lib.l3m_load(os.fsencode(str(path)), C.byref(opts))
        if not handle:
            raise RuntimeError(f"could not load {path}: see the message on stderr")
        self._m = handle
        self.vocab, self.ctx = self._lib.l3m_vocab(handle), self._lib.l3m_ctx(handle)
        self.bos, self.eos = self._lib.l3m_bos(handle), self._lib.l3m_eos(handle)

    def _handle(self):
        if self._m is None:
            raise ValueError("this model was closed")
        return self._m

    def close(self):
        handle, self._m = self._m, None
        if handle:
            self._lib.l3m_free(handle)

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def describe(self):
        return self._lib.l3m_describe(self._handle()).decode()

    @property
    def persistent(self):
        """True when decode runs as the persistent kernel (else one graph per step)."""
        return bool(self._lib.l3m_decode_persistent(self._handle()))

    def generate(self, ids, max_new, temperature=0.0, seed=0, on_token=None):
        """Greedy ids after the prompt (l3m_generate); on_token(id) returning False stops early."""
        sink = _TokenSink(on_token)
        prompt = (C.c_int32 * max(len(ids), 1))(*ids)
        n = self._lib.l3m_generate(self._handle(), prompt, len(ids), max_new, temperature, seed % (1 << 64), sink.c_func, None)
        if sink.error is not None:
            raise sink.error
        if n < 0:
            raise ValueError("l3m_generate refused the call: see the message on stderr")
        if n == 0 and len(ids) >= self.ctx:
            raise ValueError(f"a prompt of {len(ids)} ids does not fit ctx {self.ctx}")
        return sink.ids

    @property
    def logits(self):
        ptr = self._lib.l3m_logits(self._handle())
        return np.ctypeslib.as_array(ptr, shape=(self.vocab,)).copy()

    @property
    def attention_mode(self):
        """The decode step's attention: 2 matrix cores over the LDS window, 1 VALU over it, 0 from the cache."""
        return self._lib.l3m_decode_attention(self._handle())

    @property
    def window(self):
        """Positions the decode step's LDS K/V window holds (ctx when all fit); past it attention reads the cache."""
        return self._lib.l3m_decode_window(self._handle())

    def kv_rows(self, layer, kvh, pos0, n, hd=None):
        """bf16 K and V rows [pos0, pos0 + n) of one kv head of one layer's cache, as uint16 [n, hd] each (hd is
        the model's; a different one is refused)."""
        model_hd = self._lib.l3m_head_dim(self._handle())
        if hd is not None and hd != model_hd:
            raise ValueError(f"head_dim {hd} is not the model's {model_hd}")
        hd = model_hd
        k, v = np.zeros((n, hd), np.uint16), np.zeros((n, hd), np.uint16)
        if self._lib.l3m_kv_rows(self._handle(), layer, kvh, pos0, n, _p(k), _p(v)) != 0:
            raise ValueError("K/V rows out of range")
        return k, v

    @property
    def prefilled(self):
        """Prompt positions the last generate call ran as one batched prefill."""
        return self._lib.l3m_prefill_positions(self._handle())

    def logits_at(self, pos):
        """The logits the last generate computed at position pos (within its last 128 positions)."""
        out = np.empty(self.vocab, np.float32)
        if self._lib.l3m_logits_at(self._handle(), pos, out.ctypes.data_as(_f)) != 0:
            raise ValueError(f"no logits kept for position {pos}")
        return out

    def step_layout(self):
        """The decode step's geometry: head groups, FFN chunks, query heads per group, rows per chunk, head
        tiles per head workgroup (l3m_step_layout)."""
        out = (C.c_int * 5)()
        self._lib.l3m_step_layout(self._handle(), out)
        return dict(zip(("groups", "chunks", "nq", "chunk", "head_tpw"), out))

    def step_matvec(self, which, layer, index, x, rows):
        """One matvec of the decode step on its own stored matrix and in its own form (l3m_step_matvec):
        which 0 q/k/v of group index, 1 its Wo, 2 gate/up of chunk index, 3 its Wdown, 4 the head."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float32)
        if self._lib.l3m_step_matvec(self._handle(), which, layer, index, x.ctypes.data_as(_f), y.ctypes.data_as(_f)) != 0:
            raise RuntimeError(f"l3m_step_matvec({which}, {layer}, {index}) failed")
        return y

    def encode(self, text, bos=True):
        raw = text.encode()
        cap = len(raw) + 2
        out = (C.c_int32 * cap)()
        n = self._lib.l3m_encode(self._handle(), raw, int(bos), out, cap)
        return list(out[:n])

    def decode_bytes(self, ids):
        size = C.c_int()
        parts = []
        for t in ids:
            ptr = self._lib.l3m_decode(self._handle(), t, C.byref(size))
            parts.append(C.string_at(ptr, size.value))
        return b"".join(parts)

    def perf(self):
        counters = Perf()
        ok = self._lib.l3m_perf_read(self._handle(), C.byref(counters)) == 0
        return {n: (getattr(counters, n) if ok else float("nan")) for n in PERF_FIELDS}

    def bench_decode(self, prompt, n_tokens):
        """Seconds per generated token over n_tokens greedy tokens, restarting at a full context."""
        arr = (C.c_int32 * len(prompt))(*prompt)
        ns = self._lib.l3m_bench_decode(self._handle(), arr, len(prompt), n_tokens)
        if ns < 0:
            raise RuntimeError("bench_decode failed")
        return ns * 1e-9


# ------------------------------------------------------------------------------- synthetic models

@dataclass(frozen=True)
class Config:
    name: str
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn_dim: int
    vocab: int
    ctx: int
    dtype: str
    n_prompt: int = 4


# The BASELINE configurations (random-init N(0, 0.02), RoPE theta 1e4, eps 1e-5, tied head of the body dtype).
CONFIGS = {
    "stories15M": Config("stories15M", 288, 6, 6, 6, 768, 32000, 256, "bf16"),
    "stories42M": Config("stories42M", 512, 8, 8, 8, 1376, 32000, 1024, "q8_0"),
    "stories110M": Config("stories110M", 768, 12, 12, 12, 2048, 32000, 128, "q4_0"),
    "smollm2": Config("smollm2", 576, 30, 9, 3, 1536, 49152, 256, "q8_0", n_prompt=64),
}


def write_model(path, cfg, dtype=None, seed=1, std=0.02, norm_jitter=0.0, tied=True, head_dtype=None, arch="llama"):
    """Write the seeded synthetic model of cfg (a Config or a name) to path. arch "gpt2" writes the GPT-2
    variant: LayerNorm with biases, learned positions, a GELU MLP without gate, biases on every matrix;
    "gptneo" the same without the q, k, v biases."""
    cfg = CONFIGS[cfg] if isinstance(cfg, str) else cfg
    dt = DTYPES[dtype or cfg.dtype]
    spec = GenSpec(arch=arch.encode(), dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                   ffn_dim=cfg.ffn_dim, vocab=cfg.vocab, ctx=cfg.ctx, rope_theta=10000.0, norm_eps=1e-5, dtype=dt,
                   head_dtype=DTYPES[head_dtype] if head_dtype else dt, tied=int(tied), seed=seed, std=std,
                   norm_jitter=norm_jitter, bos=-1, eos=-1)
    if lib().l3m_gen_write(C.byref(spec), os.fsencode(str(path))):
        raise OSError(f"could not write {path}")
    return Path(path)


def prompt(seed, vocab, n):
    out = (C.c_int32 * n)()
    lib().l3m_gen_prompt(seed, vocab, n, out)
    return list(out)


def quantize_rows(dtype, x):
    """ggml round-to-nearest rows, as the exporter writes them: float32 [n, k] -> uint8 [n, row_bytes]."""
    x = np.ascontiguousarray(x, np.float32)
    n, k = x.shape
    rb = {F32: 4 * k, BF16: 2 * k}.get(dtype) or k // 32 * BLOCK_BYTES[dtype]
    out = np.zeros((n, rb), np.uint8)
    for i in range(n):
        lib().l3m_quantize_row(dtype, _p(out[i]), _p(x[i], _f), k)
    return out


# ---------------------------------------------------------------------------------- device level

class Device:
    """Device memory and single kernels on the library's stream (numpy in, numpy out)."""

    def __init__(self):
        self.lib = lib()
        if self.lib.l3m_dev_init():
            err = self.lib.l3m_dev_error()
            raise RuntimeError(f"no usable HIP device: {err.decode() if err else '?'}")
        self._live = []

    def _check(self, rc, what):
        if rc:
            err = self.lib.l3m_dev_error()
            raise RuntimeError(f"{what}: {err.decode() if err else 'device error'}")

    def alloc(self, nbytes):
        p = self.lib.l3m_dev_alloc(nbytes)
        if not p:
            raise MemoryError(f"device alloc of {nbytes} bytes")
        self._live.append(p)
        return p

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = self.alloc(max(a.nbytes, 16))
        self._check(self.lib.l3m_dev_upload(p, _p(a), a.nbytes), "upload")
        return p

    def get(self, p, shape, dtype):
        out = np.zeros(shape, dtype)
        self._check(self.lib.l3m_dev_download(_p(out), p, out.nbytes), "download")
        return out

    def free_all(self):
        self.lib.l3m_dev_sync()
        for p in self._live:
            self.lib.l3m_dev_free(p)
        self._live = []

    def pack_rows(self, dtype, rows, k):
        """File rows (uint8 [n, row_bytes] or a list with None for zero rows) -> host lane-tile planes."""
        n = len(rows)
        qs, ss = self.lib.l3m_lt_quant_size(dtype, n, k), self.lib.l3m_lt_scale_size(dtype, n, k)
        q, s = np.zeros(qs, np.uint8), np.zeros(max(ss, 1), np.uint8)
        keep = [None if r is None else np.ascontiguousarray(r, np.uint8) for r in rows]
        ptrs = (C.c_void_p * n)(*[None if r is None else r.ctypes.data for r in keep])
        self.lib.l3m_lt_pack_rows(dtype, n, k, ptrs, _p(q), _p(s))
        return q, s[:ss]

    def matrix(self, dtype, rows, k):
        """Upload file rows as a device lane-tile matrix."""
        q, s = self.pack_rows(dtype, rows, k)
        m = DMat(self.put(q), self.put(s) if len(s) else None, len(rows), (len(rows) + 15) // 16, (k + 31) // 32, dtype)
        return m

    def prep(self, dtype, x):
        """Activation prep on the device: returns the raw prepared bytes (q8 | scale | sum, or bf16, or f32)."""
        x = np.ascontiguousarray(x, np.float32)
        n = self.lib.l3m_act_bytes(dtype, len(x))
        dx, da = self.put(x), self.alloc(n)
        self._check(self.lib.l3m_k_prep(dtype, dx, len(x), da, None), "prep")
        return self.get(da, n, np.uint8)

    def gemv(self, m, x):
        x = np.ascontiguousarray(x, np.float32)
        k = len(x)
        n = self.lib.l3m_act_bytes(m.dtype, k)
        dx, da, dy = self.put(x), self.alloc(n), self.alloc(m.rows * 4)
        self._check(self.lib.l3m_k_prep(m.dtype, dx, k, da, None), "prep")
        self._check(self.lib.l3m_k_gemv(C.byref(m), da, k, dy, None), "gemv")
        return self.get(dy, m.rows, np.float32)

    def attend(self, q, k, v, pos, hd, stride):
        dq, dk, dv, do = self.put(np.float32(q)), self.put(np.uint16(k)), self.put(np.uint16(v)), self.alloc(hd * 4)
        self._check(self.lib.l3m_k_attend(do, dq, dk, dv, pos, hd, stride, None), "attend")
        return self.get(do, hd, np.float32)

    def rmsnorm(self, x, w, eps):
        x = np.float32(x)
        dy = self.alloc(x.nbytes)
        self._check(self.lib.l3m_k_rmsnorm(dy, self.put(x), self.put(np.float32(w)), len(x), eps, None), "rmsnorm")
        return self.get(dy, len(x), np.float32)

    def rope(self, v, n_heads, hd, pos, theta, ctx=None):
        ctx = ctx or pos + 1
        table = np.zeros(ctx * hd, np.float32)
        self.lib.l3m_rope_table(_p(table, _f), ctx, hd, theta)
        dv = self.put(np.float32(v))
        self._check(self.lib.l3m_k_rope(dv, n_heads, hd, pos, self.put(table), None), "rope")
        return self.get(dv, len(v), np.float32)

    def silu_mul(self, h, g):
        dh = self.put(np.float32(h))
        self._check(self.lib.l3m_k_silu_mul(dh, self.put(np.float32(g)), len(h), None), "silu_mul")
        return self.get(dh, len(h), np.float32)

    def dequant(self, m, row0, n):
        """Rows [row0, row0 + n) of device matrix m through the decode step's dequantization: float32 [n, 32 nb]."""
        out = self.alloc(n * m.nb * 32 * 4)
        self._check(self.lib.l3m_k_dequant(C.byref(m), row0, n, out, None), "dequant")
        return self.get(out, (n, m.nb * 32), np.float32)

    def attend_decode(self, mode, q, kc, vc, nq, nkv, hd, ctx, pos):
        """One head group's decode attention (mode 2 matrix cores, 1 LDS window, 0 cache): out [nq, hd]."""
        do = self.alloc(nq * hd * 4)
        self._check(self.lib.l3m_k_attend_decode(mode, do, self.put(np.float32(q)), self.put(np.uint16(kc)), self.put(np.uint16(vc)),
                                                 nq, nkv, hd, ctx, pos, None), "attend_decode")
        return self.get(do, (nq, hd), np.float32)

    def argmax(self, x):
        do = self.alloc(4)
        self._check(self.lib.l3m_k_argmax(self.put(np.float32(x)), len(x), do, None), "argmax")
        return int(self.get(do, 1, np.int32)[0])
