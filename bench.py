#!/usr/bin/env python3
"""Batch-1 decode benchmark of the gfx950 backend (BASELINE.json metric: decode tok/s + matvec weight GB/s vs
roofline, per dtype).

Headline (value): greedy decode of the stories110M-shaped q4_0 Llama (dim 768, 12 layers,
12 heads, ffn 2048, vocab 32000, ctx 128, tied q4_0 head, random-init N(0, 0.02)) from a one-token prompt
(token 0, as the reference's `l3m bench` feeds BOS or 0, main.c:244), restarted when the context fills
(main.c:247-251). A step is one generated token; exactly --steps are timed, after --warmup. Weights are
resident in HBM before the timed region. One JSON line on stdout:
  value / ms_per_step  generated tokens per second over the timed tokens (wall clock around the run)
  roofline             the decode kernel (k_decode, one persistent launch per run of up to 64 forward
                       passes): the algorithmic bytes of the passes it ran (body weights every pass, head
                       weights on passes with logits, K/V rows read and written) over its launch durations
                       (hipEvents around each launch on the library stream), against 8 TB/s HBM3E;
                       traffic = HBM bytes per launch from the committed rocprofv3 counter profile
  decode               one line per BASELINE decode configuration and dtype (C1 stories15M bf16, C3
                       stories42M q8_0 at ctx 1024, C4 stories110M q4_0, C5 SmolLM2-135M q8_0 and mxfp4 with
                       the 64-token prompt prefilled): 256 greedy tokens, restarting at a full context, median
                       of 5 GPU runs; k_decode's roofline fraction; the reference's own engine on this host
                       (median of 7 runs, cores and ISA stated); C5 also times the prompt to its first logits
  matvec               per dtype at the microbench shapes: warm (one matrix re-read) and
                       cold (round robin over > 512 MiB of copies) GB/s, each against 8 TB/s and against a
                       streaming read of the same bytes in the same residency (the measured roofline), with
                       the reference's own matvec table on one core and on all physical cores
  cpu_baseline         the reference (oracle/_ref, built from its sources) on the headline workload: median
                       of 7 runs of --steps tokens on this host's physical cores (at most 16)
"""
import argparse
import ctypes as C
import json
import math
import os
import statistics
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
KINDS = ["attn_block", "ffn_block", "head"]
MICRO_SHAPES = [(288, 768), (768, 288), (2048, 768), (4096, 4096), (14336, 4096)]
# README.md:52-56 of the reference (Ryzen 9 7950X, median of 7 runs of 256 tokens, real weights)
PUBLISHED = {("stories110M", "q4_0"): 5800.0, ("stories15M", "bf16"): 15300.0, ("stories42M", "q8_0"): 10700.0,
             ("smollm2", "q8_0"): 530.0}
# (config, dtype, ctx, prompt kind): BASELINE configs 1, 3, 4 and 5
DECODE_LINES = [("stories15M", "bf16", 0, "seeded"), ("stories42M", "q8_0", 1024, "seeded"), ("stories110M", "q4_0", 0, "bos"),
                ("smollm2", "q8_0", 0, "seeded"), ("smollm2", "mxfp4", 0, "seeded")]
N_TOKENS = 256


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prompt_of(A, cfg, kind):
    return [0] if kind == "bos" else A.prompt(1, cfg.vocab, cfg.n_prompt)


def decode_bytes(A, m, cfg, work):
    """Algorithmic bytes of `work` = (forward passes, passes with the head, K/V rows read per kv head and
    layer): the weight bytes of the file's blocks (rows x k x bytes per weight, as the reference's
    bytes_token, engine.c:591) and the bf16 K/V rows read and written."""
    lib, h = A.lib(), m._handle()
    body = cfg.n_layers * (lib.l3m_kernel_bytes(h, 0, 0) + lib.l3m_kernel_bytes(h, 1, 0))
    head = lib.l3m_kernel_bytes(h, 2, 0)
    row = cfg.n_layers * cfg.n_kv_heads * 2 * (cfg.dim // cfg.n_heads) * 2      # K and V, bf16, every layer
    steps, head_steps, kv_rows = work
    return steps * body + head_steps * head + kv_rows * row + steps * row


class DecodeTimer:
    """k_decode's launches (hipEvents on the library stream) and the work they did, over a region."""

    def __init__(self, A, m):
        self.A, self.m, self.lib = A, m, A.lib()

    def __enter__(self):
        self.lib.l3m_dev_sync()
        self.w0 = (C.c_double * 3)()
        self.lib.l3m_decode_work(self.m._handle(), self.w0)
        self.lib.l3m_decode_timer(1, None, None)
        return self

    def __exit__(self, *exc):
        self.lib.l3m_dev_sync()
        us, launches = C.c_double(), C.c_int()
        self.lib.l3m_decode_timer(0, C.byref(us), C.byref(launches))
        w1 = (C.c_double * 3)()
        self.lib.l3m_decode_work(self.m._handle(), w1)
        self.us, self.launches = us.value, launches.value
        self.work = [w1[i] - self.w0[i] for i in range(3)]

    def roofline(self, cfg):
        if not (self.m.persistent and self.launches):
            return None
        nbytes = decode_bytes(self.A, self.m, cfg, self.work)
        gbs = nbytes / (self.us * 1e3)
        return {"kernel": "k_decode", "launches": self.launches, "steps": self.work[0], "head_steps": self.work[1],
                "us": self.us / self.launches, "bytes": nbytes / self.launches, "GBs": gbs, "us_per_step": self.us / self.work[0]}


def measured_traffic(cfg_name, dtype, kernel, steps_per_launch=None):
    """HBM bytes per launch of a kernel (read + written), from the committed counter profile of this
    configuration (profiles/decode_<config>_<dtype>_traffic.json: two rocprofv3 --pmc passes, FETCH_SIZE
    and WRITE_SIZE, scaled by the plain copy kernel's readings). k_decode's entry is per forward pass (its
    launches run different numbers of passes), scaled here by this run's passes per launch. None when no
    profile covers it."""
    p = ROOT / "profiles" / f"decode_{cfg_name}_{dtype}_traffic.json"
    if not p.exists():
        return None
    k = json.loads(p.read_text())["kernels"].get(kernel if kernel.startswith("k_") else "k_" + kernel)
    if k is None:
        return None
    if "read_bytes_per_step" in k:
        return None if steps_per_launch is None else round((k["read_bytes_per_step"] + k["write_bytes_per_step"]) * steps_per_launch)
    return k["read_bytes"] + k["write_bytes"]


def host_cores():
    """One CPU per physical core of this process's affinity, at most 16 (the box's share for one GPU)."""
    seen, cpus = set(), []
    for c in sorted(os.sched_getaffinity(0)):
        try:
            t = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
            key = ((t / "physical_package_id").read_text().strip(), (t / "core_id").read_text().strip())
        except OSError:
            key = (c,)
        if key not in seen:
            seen.add(key)
            cpus.append(c)
    return cpus[:16]


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def tokens_per_run(model, prompt, n, restart):
    """Generate n tokens from prompt, restarting when the context fills (main.c:247-251); returns the count."""
    done = 0
    while done < n:
        got = len(model.generate(prompt, n - done))
        if got == 0:
            break
        done += got
        if not restart:
            break
    return done


def cpu_decode(path, prompt, n_tokens, ctx, runs=7):
    """The reference's own engine (oracle/_ref, its CPUID-picked AVX2/AVX-512 table) on this host's physical
    cores: one warm-up, then the median of `runs` runs of n_tokens greedy tokens (README.md:58-62)."""
    from oracle.oracle import Reference
    if not Reference.available():
        return None
    os.environ.pop("L3M_ISA", None)
    cpus = host_cores()
    m = Reference().load(path, ctx=ctx, cpus=cpus)
    tokens_per_run(m, prompt, min(n_tokens, 32), True)
    rates = []
    for _ in range(runs):
        t0 = time.perf_counter()
        n = tokens_per_run(m, prompt, n_tokens, True)
        rates.append(n / (time.perf_counter() - t0))
    desc = m.describe()
    return {"value": round(statistics.median(rates), 1), "unit": "tok/s", "cores": len(cpus), "kind": "reference",
            "sample": f"median of {runs} runs of {n_tokens} greedy tokens after one warm-up (min {min(rates):.0f}, max {max(rates):.0f}), "
                      f"same model file and prompt, restarts at the full context; {desc}; {cpu_model()}"}


def cpu_first_logits(path, prompt, ctx, runs=3):
    """Milliseconds from the prompt to its first logits on the reference's engine (token by token)."""
    from oracle.oracle import Reference
    if not Reference.available():
        return None
    m = Reference().load(path, ctx=ctx, cpus=host_cores())
    m.generate(prompt, 0)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        m.generate(prompt, 0)
        times.append((time.perf_counter() - t0) * 1e3)
    return round(statistics.median(times), 3)


def gpu_first_logits(A, path, prompt, ctx, reps=5):
    """Milliseconds to the first logits of the prompt on the GPU, median of reps after one call: batched
    prefill replaying its captured graph (and the first call, which captures it), the same launches one by
    one (L3M_PREFILL_GRAPH=0), and token by token (L3M_PREFILL=0)."""
    out = {}
    for key, env in (("ms_prefill", {}), ("ms_prefill_loose_launches", {"L3M_PREFILL_GRAPH": "0"}),
                     ("ms_token_by_token", {"L3M_PREFILL": "0"})):
        for k in ("L3M_PREFILL", "L3M_PREFILL_GRAPH"):
            os.environ.pop(k, None)
        os.environ.update(env)
        with A.Model(path, ctx=ctx) as m:
            t0 = time.perf_counter()
            m.generate(prompt, 0)
            A.lib().l3m_dev_sync()
            first = (time.perf_counter() - t0) * 1e3
            times = []
            for _ in range(reps):
                t0 = time.perf_counter()
                m.generate(prompt, 0)
                A.lib().l3m_dev_sync()
                times.append((time.perf_counter() - t0) * 1e3)
            out[key] = round(statistics.median(times), 3)
            if not env:
                out["ms_prefill_first_call"] = round(first, 3)
                out["prefilled_positions"] = m.prefilled
    for k in ("L3M_PREFILL", "L3M_PREFILL_GRAPH"):
        os.environ.pop(k, None)
    return out


def decode_line(A, d, name, dtype, ctx, kind, cpu_runs, gpu_runs=5):
    cfg = A.CONFIGS[name]
    path = A.write_model(Path(d) / f"{name}-{dtype}.l3m", cfg, dtype=dtype, seed=1)
    prompt = prompt_of(A, cfg, kind)
    with A.Model(path, ctx=ctx) as m:
        m.bench_decode(prompt, 32)
        rates, dom = [], None
        with DecodeTimer(A, m) as t:
            for _ in range(gpu_runs):
                rates.append(1.0 / m.bench_decode(prompt, N_TOKENS))
        dom = t.roofline(cfg)
        wbytes = A.lib().l3m_weight_bytes(m._handle())
        mctx, persistent, att = m.ctx, m.persistent, m.attention_mode
    value = statistics.median(rates)
    line = {"config": name, "dtype": dtype, "ctx": mctx, "prompt_tokens": len(prompt), "tokens": N_TOKENS,
            "value": round(value, 1), "unit": "tok/s", "us_per_token": round(1e6 / value, 2),
            "gpu_runs": [round(r, 1) for r in rates], "persistent": persistent, "attention_mode": att,
            "weight_bytes_per_token": wbytes, "weight_GBs": round(wbytes * value * 1e-9, 1)}
    if dom:
        line["roofline"] = {"bound": "hbm", "kernel": "k_decode", "achieved": round(dom["GBs"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": round(dom["GBs"] / PEAK_HBM_GBS, 4), "us_per_step": round(dom["us_per_step"], 2)}
    pub = PUBLISHED.get((name, dtype))
    line["published"] = pub
    line["vs_published"] = round(value / pub, 3) if pub else None
    if len(prompt) > 8:
        line["first_logits"] = gpu_first_logits(A, path, prompt, ctx)
    if cpu_runs:
        line["cpu_baseline"] = cpu_decode(path, prompt, N_TOKENS, ctx, cpu_runs)
        if line["cpu_baseline"]:
            line["vs_cpu"] = round(value / line["cpu_baseline"]["value"], 3)
            if len(prompt) > 8:
                line["first_logits"]["cpu_ms"] = cpu_first_logits(path, prompt, ctx)
    log(f"decode {name} {dtype} ctx {mctx}: {line['value']} tok/s ({line['us_per_token']} us/token, "
        f"k_decode {line.get('roofline', {}).get('us_per_step', '-')} us/pass, {line.get('roofline', {}).get('frac', '-')} of HBM peak); "
        f"cpu {line.get('cpu_baseline', {}) and line['cpu_baseline']['value']} tok/s")
    return line


def cpu_matvec_lib():
    p = ROOT / "oracle" / "_ref" / "libcpubench.so"
    if not p.exists():
        return None
    lib = C.CDLL(str(p))
    lib.cb_gemv_gbs.restype = C.c_double
    lib.cb_gemv_gbs.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_double]
    lib.cb_table.restype = C.c_int
    return lib


def matvec_bench(A, dtypes, iters=50, cpu_seconds=0.2, shapes=None):
    """Warm: one matrix re-read; cold: round robin over copies totalling > 512 MiB (beyond the 256 MB
    Infinity Cache). Launches run back to back and each figure is their mean interval; where the warm
    matvec or read is within 1.5x of an empty kernel's launch interval, warm_launch_bound marks it (those
    warm figures are the launch rate). Beside each, the measured roofline (a streaming read of the same bytes, warm and cold)
    and the reference's own matvec table (tests/test_kernels.c:151-176's method) on one core and on all."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from weights import rows as make_rows
    lib, dev, cpu = A.lib(), A.Device(), cpu_matvec_lib() if cpu_seconds > 0 else None
    cores = host_cores()
    arr = (C.c_int * len(cores))(*cores)
    # back-to-back launches of an empty kernel: a warm figure within 1.5x of this interval is the launch
    # rate of a short kernel, not its duration (the committed kernel trace has the durations)
    interval = lib.l3m_time_launch_interval(200)
    out = {"launch_interval_us": round(interval, 3)}
    for name in dtypes:
        dt = A.DTYPES[name]
        res = {}
        for n, k in shapes or MICRO_SHAPES:
            w = make_rows(dt, n, k, seed=n + k)
            x = np.random.default_rng(0).standard_normal(k).astype(np.float32)
            q, s = dev.pack_rows(dt, w, k)
            nbytes = len(q) + len(s)
            copies = 1 + (512 << 20) // nbytes
            mats = (A.DMat * copies)()
            dq = dev.put(np.tile(q, copies))                      # each copy starts 256-byte aligned
            ds = dev.put(np.tile(s, copies)) if len(s) else None
            for i in range(copies):
                mats[i] = A.DMat(dq + i * len(q), ds + i * len(s) if ds else None, n, (n + 15) // 16, (k + 31) // 32, dt)
            act = dev.alloc(lib.l3m_act_bytes(dt, k))
            lib.l3m_k_prep(dt, dev.put(x), k, act, None)
            y = dev.alloc(n * 4)
            warm = lib.l3m_time_gemv(mats, 1, act, k, y, iters)
            cold = lib.l3m_time_gemv(mats, copies, act, k, y, max(iters, 2 * copies))
            rb = (nbytes + 16 + 15) // 16 * 16                   # read roofline: the same bytes (+ its scratch word)
            rcopies = 1 + (512 << 20) // rb
            rbuf = dev.alloc(rb * rcopies)
            bufs = (C.c_void_p * rcopies)(*[rbuf + i * rb for i in range(rcopies)])
            rwarm = lib.l3m_time_read(bufs, 1, rb, iters)
            rcold = lib.l3m_time_read(bufs, rcopies, rb, max(iters, 2 * rcopies))
            r = {"bytes": nbytes, "warm_us": round(warm, 3), "warm_GBs": round(nbytes / warm * 1e-3, 1),
                 "cold_us": round(cold, 3), "cold_GBs": round(nbytes / cold * 1e-3, 1),
                 "cold_frac_of_peak": round(nbytes / cold * 1e-3 / PEAK_HBM_GBS, 3),
                 "read_warm_GBs": round(nbytes / rwarm * 1e-3, 1), "read_cold_GBs": round(nbytes / rcold * 1e-3, 1),
                 "warm_frac_of_read": round(rwarm / warm, 3), "cold_frac_of_read": round(rcold / cold, 3),
                 "warm_launch_bound": bool(min(warm, rwarm) < 1.5 * interval)}
            if cpu:
                wc = np.ascontiguousarray(w)
                r["cpu_1core_GBs"] = round(cpu.cb_gemv_gbs(dt, n, k, wc.ctypes.data, x.ctypes.data, arr, 1, cpu_seconds), 1)
                r["cpu_all_GBs"] = round(cpu.cb_gemv_gbs(dt, n, k, wc.ctypes.data, x.ctypes.data, arr, len(cores), cpu_seconds), 1)
            res[f"{n}x{k}"] = r
            dev.free_all()
        out[name] = res
        log(f"matvec {name} (GB/s warm/cold | read roofline warm/cold | cpu 1/{len(cores)} cores): " +
            ", ".join(f"{s} {r['warm_GBs']:.0f}/{r['cold_GBs']:.0f} | {r['read_warm_GBs']:.0f}/{r['read_cold_GBs']:.0f} | "
                      f"{r.get('cpu_1core_GBs', '-')}/{r.get('cpu_all_GBs', '-')}" for s, r in res.items()))
    if cpu:
        out["cpu"] = {"table": ["scalar", "avx2", "avx512"][cpu.cb_table()], "cores": len(cores), "model": cpu_model(),
                      "method": f"the reference's own gemv table on its packed tiles, looped for {cpu_seconds} s, warm (resident), "
                                "one core, then every core on a contiguous range of tiles"}
    return out


def sampled_rate(A, m, prompt, n_tokens, temperature=1.0):
    """Tokens/s of the same decode loop with temperature sampling on the device (l3m_bench_decode_t);
    a side figure (the metric is greedy decode)."""
    lib, arr = A.lib(), (C.c_int32 * len(prompt))(*prompt)
    lib.l3m_bench_decode_t(m._handle(), arr, len(arr), 32, temperature, 0)
    ns = lib.l3m_bench_decode_t(m._handle(), arr, len(arr), n_tokens, temperature, 1)
    return {"temperature": temperature, "value": round(1e9 / ns, 1) if ns > 0 else None, "unit": "tok/s"}


def streamed_rate(A, m, prompt, n_tokens):
    """Tokens/s of greedy generate calls with an on_token callback (tokens handed over as they come: runs of
    8 positions, two in flight), restarting at a full context; a side figure beside the headline's runs of
    up to 128 positions. The Python callback's own cost per token is included."""
    m.generate(prompt, 16, on_token=lambda t: True)
    t0, done = time.perf_counter(), 0
    while done < n_tokens:
        got = m.generate(prompt, min(n_tokens - done, m.ctx - len(prompt)), on_token=lambda t: True)
        if not got:
            break
        done += len(got)
    return {"value": round(done / (time.perf_counter() - t0), 1), "unit": "tok/s", "tokens": done}


def cold_rate(A, path, prompt, n_tokens):
    """Tokens/s with the caches emptied of the weights before every forward pass (--cold, engine.c:330-338),
    the eviction not counted: a side figure (README.md:46-47 reports 6-8x slower on the CPU)."""
    with A.Model(path, cold=True) as m:
        m.bench_decode(prompt, 8)
        return {"value": round(1.0 / m.bench_decode(prompt, n_tokens), 1), "unit": "tok/s", "tokens": n_tokens}


A_PHASES = ["weights issued", "wait", "prologue", "norm+prep", "qkv", "rope+kv", "attention", "prep", "wo", "write", "flag"]
F_PHASES = ["weights issued", "wait", "prologue", "norm+prep", "gate/up", "rows", "silu+prep", "down", "write", "flag"]


def phase_report(A, d, name, dtype, pos, layer):
    """Per-phase durations of the decode step (the library built with L3M_PHASE_STAMPS): for layers
    (layer, layer + 1) at position pos, each phase's median and largest duration over the attention groups
    and the FFN chunks, the hand-overs between them, and the layer's span, in microseconds. For the last
    layer the second layer is layer 0 of position pos + 1, and the report adds the step's tail through the
    head (head_chain_us)."""
    import numpy as np
    lib, cfg = A.lib(), A.CONFIGS[name]
    path = A.write_model(Path(d) / f"{name}-{dtype}-phases.l3m", cfg, dtype=dtype, seed=1)
    prompt = [0]
    with A.Model(path) as m:
        m.bench_decode(prompt, 64)
        if lib.l3m_phase_stamps(0, pos, layer, None):
            raise RuntimeError("phase stamps unavailable: run with the library built by `make -C l3m_amd/csrc phases`")
        m.generate(prompt, min(pos + 8, cfg.ctx - 2))
        lib.l3m_dev_sync()
        out, clk = np.zeros((2, 192, 16), np.uint64), np.zeros((2, 192, 16), np.uint64)
        lib.l3m_phase_stamps(1, pos, layer, out.ctypes.data)
        lib.l3m_phase_stamps(2, pos, layer, clk.ctypes.data)
    t = out.astype(np.float64) * 0.01                 # 100 MHz ticks -> us
    groups = [g for g in range(64) if t[0, g, 1] > 0]
    chunks = [c for c in range(64, 128) if t[0, c, 1] > 0]

    def spans(rows, names, lay):
        res = {}
        for e in range(1, len(names)):
            v = [t[lay, r, e] - t[lay, r, e - 1] for r in rows if t[lay, r, e] > 0 and t[lay, r, e - 1] > 0]
            if v:
                res[names[e]] = {"median": round(float(np.median(v)), 3), "max": round(float(np.max(v)), 3)}
        return res

    a_done = max(t[0, g, 10] for g in groups)
    f_start = min(t[0, c, 1] for c in chunks)
    f_done = max(t[0, c, 9] for c in chunks)
    a_next = min(t[1, g, 1] for g in groups) if all(t[1, g, 1] > 0 for g in groups) else None
    rep = {"config": name, "dtype": dtype, "pos": pos, "layer": layer, "attention_groups": len(groups), "ffn_chunks": len(chunks),
           "attention": spans(groups, A_PHASES, 0), "ffn": spans(chunks, F_PHASES, 0),
           "attention_block_us": round(float(np.median([t[0, g, 10] - t[0, g, 1] for g in groups])), 3),
           "ffn_block_us": round(float(np.median([t[0, c, 9] - t[0, c, 1] for c in chunks])), 3),
           "handover_attention_to_ffn_us": round(float(f_start - a_done), 3),
           "handover_ffn_to_attention_us": round(float(a_next - f_done), 3) if a_next else None,
           "layer_us": round(float(np.median([t[1, g, 1] - t[0, g, 1] for g in groups])), 3) if a_next else None}
    # the shader clock over attention group 0's block: s_memtime ticks per microsecond of the 100 MHz clock
    g0 = groups[0]
    rep["shader_clock_mhz"] = round(float((clk[0, g0, 10].astype(np.float64) - clk[0, g0, 1]) / (t[0, g0, 10] - t[0, g0, 1])), 1)
    heads = [h for h in range(128, 192) if t[1 if layer + 1 == cfg.n_layers - 1 else 0, h, 1] > 0]
    if heads:
        lay = 1 if layer + 1 == cfg.n_layers - 1 else 0
        rep["head"] = {"wait_to_block_end_median": round(float(np.median([t[lay, h, 2] - t[lay, h, 1] for h in heads])), 3)}
    if layer == cfg.n_layers - 1 and heads and a_next:
        # the step's tail: from the last FFN chunk's flag of the last layer, the medians of each event up to
        # the next position's attention groups waking with the token
        z = f_done

        def med(vals):
            return round(float(np.median(vals)) - z, 3)
        rep["head_chain_us"] = {
            "head_workgroups_see_every_flag": med([t[0, h, 1] for h in heads]),
            "head_blocks_end": med([t[0, h, 2] for h in heads]),
            "head_keys_stored": med([t[0, h, 3] for h in heads]),
            "head_final_sum_done": med([t[0, h, 4] for h in heads if t[0, h, 4] > 0]),
            "head_norm_prep_done": med([t[0, h, 5] for h in heads if t[0, h, 5] > 0]),
            "head_matvec_done": med([t[0, h, 6] for h in heads if t[0, h, 6] > 0]),
            "next_position_attention_wakes": med([t[1, g, 1] for g in groups]),
            "next_position_prologue_done": med([t[1, g, 2] for g in groups]),
        }
    return rep


# the dependent steps of l3m_probe_latency, by index
LATENCY_STEPS = ["LDS hand-over (write, barrier, read, barrier)", "dependent LDS read", "64-lane DPP/permlane sum",
                 "bf16 matrix-core product 16x16x32", "barrier", "LDS write and read-back", "expf"]


def probes(A):
    """The residency and exchange probes (the GPU analogues of bench/residency.c and bench/exchange.c), and the
    latencies of the dependent steps inside one workgroup that the decode kernel's phases are built from."""
    lib, out = A.lib(), {"stream": [], "exchange": [], "graph_node_us": None}
    v = C.c_double()
    for xcds in (1, 8):
        for mib in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024):
            total = mib << 20
            per = total // (32 * xcds)
            if per < 4096 or per % 16:
                continue
            passes = max(1, (256 << 20) // total)
            if lib.l3m_probe_stream(per, xcds, 32, passes, C.byref(v)) == 0:
                out["stream"].append({"xcds": xcds, "workgroups": 32 * xcds, "working_set_mib": mib, "GBs": round(v.value, 1)})
    for same in (1, 0):
        for n in (2, 4, 8, 16, 28, 32):
            if lib.l3m_probe_exchange(n, same, 768, 2000, C.byref(v)) == 0:
                out["exchange"].append({"workgroups": n, "same_xcd": bool(same), "dim": 768, "us_per_round": round(v.value, 3)})
    if lib.l3m_probe_graph_node(256, 20, C.byref(v)) == 0:
        out["graph_node_us"] = round(v.value, 3)
    out["latency_clocks"] = []
    for which, name in enumerate(LATENCY_STEPS):
        for threads in (64, 1024):
            if lib.l3m_probe_latency(which, threads, C.byref(v)) == 0:
                out["latency_clocks"].append({"step": name, "threads": threads, "clocks": round(v.value, 1)})
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--config", default="stories110M")
    ap.add_argument("--dtype", default=None)
    ap.add_argument("--decode", type=int, default=1, help="the per-config decode lines (0 to skip)")
    ap.add_argument("--matvec", default="bf16,q8_0,q4_0,mxfp4", help="dtypes for the matvec microbench ('' to skip)")
    ap.add_argument("--cpu-runs", type=int, default=7, help="runs of the reference CPU engine per decode line (0 to skip)")
    ap.add_argument("--cpu-matvec-seconds", type=float, default=0.2, help="loop length of each CPU matvec figure (0 to skip)")
    ap.add_argument("--sample-temp", type=float, default=1.0, help="temperature of the sampled-decode side figure (0 to skip)")
    ap.add_argument("--cold", type=int, default=1, help="the --cold side figure (0 to skip)")
    ap.add_argument("--probes", action="store_true", help="run only the residency and exchange probes, one JSON line")
    ap.add_argument("--phases", default="", help="only per-phase timing of CONFIG:DTYPE:POS:LAYER (e.g. stories110M:q4_0:64:5), "
                                                "with l3m_amd/libl3m_hip_phases.so, one JSON line")
    ap.add_argument("--only-decode", action="store_true", help="the headline decode only (for profiling runs)")
    ap.add_argument("--matvec-shapes", default="", help="rowsxk,... : only these shapes in the matvec microbench (counter passes)")
    ap.add_argument("--matvec-iters", type=int, default=50, help="timed launches per matvec figure (at least 2 per copy when cold)")
    ap.add_argument("--matvec-only", action="store_true", help="only the matvec microbench, one JSON line (profiling runs "
                                                               "of the matvec kernels: no decode, no persistent launch)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run the plain copy kernel once over this many MiB (counter calibration under rocprofv3)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this backend runs one model on one GPU; --gpus {a.gpus} is not a configuration it has "
              "(one GPU's throughput is the figure; multi-GPU sharding is described, not run)", file=sys.stderr)
        sys.exit(2)

    if a.phases:
        os.environ["L3M_HIP_LIB"] = str(ROOT / "l3m_amd" / "libl3m_hip_phases.so")
    import l3m_amd as A
    if a.phases:
        name, dt, pos, layer = a.phases.split(":")
        with tempfile.TemporaryDirectory() as d:
            print(json.dumps({"phases": phase_report(A, d, name, dt, int(pos), int(layer))}), flush=True)
        return
    if a.probes:
        print(json.dumps({"probes": probes(A)}), flush=True)
        return
    if a.matvec_only:
        shapes = [tuple(int(v) for v in sh.split("x")) for sh in a.matvec_shapes.split(",") if sh]
        print(json.dumps({"matvec": matvec_bench(A, [s for s in a.matvec.split(",") if s], iters=a.matvec_iters,
                                                 cpu_seconds=a.cpu_matvec_seconds, shapes=shapes)}), flush=True)
        return
    cfg = A.CONFIGS[a.config]
    dtype = a.dtype or cfg.dtype
    lib = A.lib()
    with tempfile.TemporaryDirectory() as d:
        path = A.write_model(Path(d) / f"{cfg.name}-{dtype}.l3m", cfg, dtype=dtype, seed=1)
        prompt = [0]
        with A.Model(path) as m:
            log(f"bench: {m.describe()} on {lib.l3m_dev_name().decode()}")
            m.bench_decode(prompt, max(a.warmup, 1))
            m.perf()                                  # l3m_perf counts from here: the timed tokens only
            with DecodeTimer(A, m) as t:
                t0 = time.perf_counter()
                m.bench_decode(prompt, a.steps)
                lib.l3m_dev_sync()
                elapsed = time.perf_counter() - t0
            dom = t.roofline(cfg)
            value = a.steps / elapsed
            perf = m.perf()
            split = {k: (None if math.isnan(perf[k]) else round(perf[k], 1)) for k in ("ns_token", "ns_wait", "ns_compute")}
            log(f"bench: {a.steps} tokens in {elapsed * 1e3:.2f} ms = {value:.0f} tok/s")
            log(f"bench: l3m_perf per token: {split['ns_token']} ns, waits of attention group 0 {split['ns_wait']} ns, "
                f"compute {split['ns_compute']} ns")
            if dom:
                log(f"bench: k_decode {dom['launches']} launches, {dom['steps']:.0f} passes, {dom['us']:.1f} us per launch, "
                    f"{dom['us_per_step']:.1f} us per pass, {dom['GBs']:.1f} GB/s algorithmic")
            wbytes = lib.l3m_weight_bytes(m._handle())
            sampled = sampled_rate(A, m, prompt, a.steps, a.sample_temp) if a.sample_temp > 0 and not a.only_decode else None
            if sampled:
                log(f"bench: sampled at T={sampled['temperature']}: {sampled['value']} tok/s")
            streamed = streamed_rate(A, m, prompt, max(a.steps, N_TOKENS)) if not a.only_decode else None
            if streamed:
                log(f"bench: streamed to on_token: {streamed['value']} tok/s")
        cold = cold_rate(A, path, prompt, min(a.steps, 64)) if a.cold and not a.only_decode else None
        if cold:
            log(f"bench: --cold {cold['value']} tok/s")
        decode = None
        if a.decode and not a.only_decode:
            decode = [decode_line(A, d, *line, cpu_runs=a.cpu_runs) for line in DECODE_LINES]
        # the headline's CPU line: the reference on the same model and prompt, runs of 256 tokens (the
        # per-config line of this workload when it ran)
        same = [ln for ln in decode or [] if (ln["config"], ln["dtype"], ln["prompt_tokens"]) == (cfg.name, dtype, len(prompt))]
        cpu = same[0].get("cpu_baseline") if same else None
        if cpu is None and a.cpu_runs > 0 and not a.only_decode:
            cpu = cpu_decode(path, prompt, max(a.steps, N_TOKENS), 0, a.cpu_runs)
        if cpu:
            log(f"bench: reference CPU {cpu['value']} tok/s on {cpu['cores']} cores")
    matvec = matvec_bench(A, [s for s in a.matvec.split(",") if s], cpu_seconds=a.cpu_matvec_seconds) if a.matvec and not a.only_decode else None
    if a.copy_mib:
        dev = A.Device()
        src, dst = dev.alloc(a.copy_mib << 20), dev.alloc(a.copy_mib << 20)
        if lib.l3m_dev_copy(dst, src, a.copy_mib << 20, None) or lib.l3m_dev_sync():
            raise RuntimeError("copy kernel failed")
        dev.free_all()
        log(f"copy: {a.copy_mib} MiB")
    pub = PUBLISHED.get((cfg.name, dtype))
    line = {
        "metric": "batch-1 decode tok/s + matvec weight GB/s vs roofline, per dtype",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(elapsed * 1e3 / a.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(value / pub, 3) if pub else None, "dtype": dtype, "data": "synthetic",
        "config": {"workload": f"{cfg.name}-shaped {dtype} Llama, batch-1 greedy decode of {a.steps} tokens from a one-token "
                               f"prompt (the reference bench's), restart at ctx {cfg.ctx}",
                   "dim": cfg.dim, "layers": cfg.n_layers, "heads": cfg.n_heads, "kv_heads": cfg.n_kv_heads,
                   "ffn": cfg.ffn_dim, "vocab": cfg.vocab, "ctx": cfg.ctx, "weights": "random-init N(0,0.02), seed 1"},
        "roofline": None if not dom else {
            "bound": "hbm", "kernel": dom["kernel"], "achieved": round(dom["GBs"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(dom["GBs"] / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(cfg.name, dtype, dom["kernel"], dom["steps"] / dom["launches"]),
            "bytes_per_launch": round(dom["bytes"]), "us_per_launch": round(dom["us"], 3), "us_per_pass": round(dom["us_per_step"], 3),
            "launches": dom["launches"], "passes": dom["steps"]},
        "weight_bytes_per_token": wbytes,
        "weight_GBs_per_token": round(wbytes * value * 1e-9, 1) if wbytes else None,
        "decode": decode,
        "matvec": matvec,
        "sampled_decode": sampled,
        "streamed_decode": streamed,
        "perf_split": split,
        "cold_decode": cold,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
