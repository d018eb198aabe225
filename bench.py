#!/usr/bin/env python3
"""Batch-1 decode benchmark of the gfx950 backend (BASELINE.json metric: decode tok/s + matvec weight GB/s
vs roofline, per dtype).

A step is one greedy decode token of the stories110M-shaped q4_0 Llama (dim 768, 12
layers, 12 heads, ffn 2048, vocab 32000, ctx 128, tied q4_0 head, random-init N(0, 0.02)), fed a 4-token
seeded prompt and restarted when the context fills (the reference's bench loop, main.c:247-251).
Weights are resident in HBM before the timed region. One JSON line on stdout:
  value / ms_per_step  generated tokens per second over exactly --steps tokens
  roofline             the decode kernel (k_decode, one persistent launch per run of up to 64 steps): the
                       algorithmic bytes of the steps it ran (body weights every step, head weights on steps
                       with logits, K/V rows read and written) over its average launch duration (hipEvents
                       around each launch on the library stream), against 8 TB/s HBM3E; traffic = the HBM
                       bytes per launch that rocprofv3 counted for the same command (profiles/)
  step_kernels         the one-graph-per-step path's three kernels, each timed alone at ctx/2
  matvec               per-dtype matvec GB/s at the microbench shapes, warm
                       (cache-resident) and cold (rotating over > 512 MiB of copies)
  cpu_baseline         fpedd/l3m itself (built from its sources into oracle/_ref), AVX2/AVX-512 path,
                       on this host's cores, same model file and prompt
"""
import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
KINDS = ["attn_block", "ffn_block", "head"]
MICRO_SHAPES = [(288, 768), (768, 288), (2048, 768), (4096, 4096), (14336, 4096)]
PUBLISHED = {("stories110M", "q4_0"): 5800.0, ("stories15M", "bf16"): 15300.0, ("stories42M", "q8_0"): 10700.0}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_table(A, m, cfg):
    lib = A.lib()
    pos = cfg.ctx // 2
    rows = []
    for kind, name in enumerate(KINDS):
        us = lib.l3m_bench_kernel(m._handle(), kind, 0, pos, 200)
        if us < 0:
            raise RuntimeError(f"timing {name} failed")
        nbytes = lib.l3m_kernel_bytes(m._handle(), kind, pos)
        per_tok = 1 if name == "head" else cfg.n_layers
        rows.append({"kernel": name, "us": us, "bytes": nbytes, "GBs": nbytes / us * 1e-3, "launches_per_token": per_tok,
                     "us_per_token": us * per_tok})
    return rows


def matvec_bench(A, dtypes, iters=50):
    """Warm: one matrix re-read; cold: round robin over copies totalling > 512 MiB (beyond the 256 MB MALL)."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from weights import rows as make_rows
    lib, dev = A.lib(), A.Device()
    out = {}
    for name in dtypes:
        dt = A.DTYPES[name]
        res = {}
        for n, k in MICRO_SHAPES:
            w = make_rows(dt, n, k, seed=n + k)
            q, s = dev.pack_rows(dt, w, k)
            nbytes = len(q) + len(s)
            copies = 1 + (512 << 20) // nbytes
            mats = (A.DMat * copies)()
            dq = dev.put(np.tile(q, copies))                      # each copy starts 256-byte aligned
            ds = dev.put(np.tile(s, copies)) if len(s) else None
            for i in range(copies):
                mats[i] = A.DMat(dq + i * len(q), ds + i * len(s) if ds else None, n, (n + 15) // 16, (k + 31) // 32, dt)
            x = np.random.default_rng(0).standard_normal(k).astype(np.float32)
            act = dev.alloc(lib.l3m_act_bytes(dt, k))
            lib.l3m_k_prep(dt, dev.put(x), k, act, None)
            y = dev.alloc(n * 4)
            warm = lib.l3m_time_gemv(mats, 1, act, k, y, iters)
            cold = lib.l3m_time_gemv(mats, copies, act, k, y, max(iters, 2 * copies))
            res[f"{n}x{k}"] = {"bytes": nbytes, "warm_us": round(warm, 3), "warm_GBs": round(nbytes / warm * 1e-3, 1),
                               "cold_us": round(cold, 3), "cold_GBs": round(nbytes / cold * 1e-3, 1),
                               "cold_frac_of_peak": round(nbytes / cold * 1e-3 / PEAK_HBM_GBS, 3)}
            dev.free_all()
        out[name] = res
        log(f"matvec {name}: " + ", ".join(f"{s} {r['warm_GBs']:.0f}/{r['cold_GBs']:.0f} GB/s" for s, r in res.items()))
    return out


def decode_bytes(A, m, cfg, work):
    """Algorithmic bytes of `work` = (steps, steps with the head, K/V rows read per kv head and layer)."""
    lib, h = A.lib(), m._handle()
    body = cfg.n_layers * (lib.l3m_kernel_bytes(h, 0, 0) + lib.l3m_kernel_bytes(h, 1, 0))
    head = lib.l3m_kernel_bytes(h, 2, 0)
    row = cfg.n_layers * cfg.n_kv_heads * 2 * (cfg.dim // cfg.n_heads) * 2      # K and V, bf16, every layer
    steps, head_steps, kv_rows = work
    return steps * body + head_steps * head + kv_rows * row + steps * row


def measured_traffic(cfg_name, dtype, kernel, steps_per_launch=None):
    """HBM bytes per launch of a kernel (read + written), from the committed counter profile of this
    configuration (profiles/decode_<config>_<dtype>_traffic.json: two rocprofv3 --pmc passes, FETCH_SIZE
    and WRITE_SIZE, scaled by the plain copy kernel's readings). k_decode's entry is per step (its launches
    run different step counts), scaled here by this run's steps per launch. None when no profile covers it."""
    p = ROOT / "profiles" / f"decode_{cfg_name}_{dtype}_traffic.json"
    if not p.exists():
        return None
    k = json.loads(p.read_text())["kernels"].get(kernel if kernel.startswith("k_") else "k_" + kernel)
    if k is None:
        return None
    if "read_bytes_per_step" in k:
        return None if steps_per_launch is None else round((k["read_bytes_per_step"] + k["write_bytes_per_step"]) * steps_per_launch)
    return k["read_bytes"] + k["write_bytes"]


def copy_calibration(A, nbytes):
    """One launch of the plain copy kernel over nbytes (read nbytes, write nbytes), for scaling counters."""
    lib, dev = A.lib(), A.Device()
    src, dst = dev.alloc(nbytes), dev.alloc(nbytes)
    if lib.l3m_dev_copy(dst, src, nbytes, None) or lib.l3m_dev_sync():
        raise RuntimeError("copy kernel failed")
    dev.free_all()
    log(f"copy: {nbytes} bytes")


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


def cpu_baseline(path, prompt, seconds):
    """The reference's own engine (oracle/_ref, AVX2/AVX-512 per its CPUID dispatch) on this host."""
    from oracle.oracle import Reference
    if not Reference.available():
        return None
    os.environ.pop("L3M_ISA", None)
    cpus = host_cores()
    ref = Reference()
    m = ref.load(path, cpus=cpus)
    m.generate(prompt, 16)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        n += len(m.generate(prompt, 10 ** 6))
    dt = time.perf_counter() - t0
    desc = m.describe()
    return {"value": round(n / dt, 1), "unit": "tok/s", "cores": len(cpus), "kind": "reference",
            "sample": f"{n} greedy tokens in {dt:.1f} s, same model file and prompt, restarts at the full context; {desc}"}


def sampled_rate(A, m, prompt, n_tokens, temperature=1.0):
    """Tokens/s of the same decode loop with temperature sampling on the device (l3m_bench_decode_t);
    a side figure (the metric is greedy decode)."""
    lib, arr = A.lib(), (C.c_int32 * len(prompt))(*prompt)
    lib.l3m_bench_decode_t(m._handle(), arr, len(arr), 32, temperature, 0)
    ns = lib.l3m_bench_decode_t(m._handle(), arr, len(arr), n_tokens, temperature, 1)
    return {"temperature": temperature, "value": round(1e9 / ns, 1) if ns > 0 else None, "unit": "tok/s"}


def prefill_figure(A, d, reps=5):
    """Time to the first logits of the C5 workload (SmolLM2-135M-shaped q8_0, its 64-token seeded prompt):
    the batched prefill against token-by-token decode steps (L3M_PREFILL=0), median of reps; a side figure."""
    cfg = A.CONFIGS["smollm2"]
    path = A.write_model(Path(d) / "smollm2-q8_0.l3m", cfg, dtype="q8_0", seed=1)
    ids = A.prompt(1, cfg.vocab, cfg.n_prompt)
    out = {"config": "smollm2-q8_0", "prompt": len(ids)}
    for key, env in (("ms_prefill", None), ("ms_token_by_token", "0")):
        if env is None:
            os.environ.pop("L3M_PREFILL", None)
        else:
            os.environ["L3M_PREFILL"] = env
        m = A.Model(path)
        m.generate(ids, 0)
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            m.generate(ids, 0)
            A.lib().l3m_dev_sync()
            times.append((time.perf_counter() - t0) * 1e3)
        out[key] = round(sorted(times)[reps // 2], 3)
        if env is None:
            out["prefilled_positions"] = m.prefilled
        m.close()
    os.environ.pop("L3M_PREFILL", None)
    return out


def probes(A):
    """The residency and exchange probes: rows of printable results."""
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
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--config", default="stories110M")
    ap.add_argument("--dtype", default=None)
    ap.add_argument("--matvec", default="bf16,q8_0,q4_0,mxfp4", help="dtypes for the matvec microbench ('' to skip)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="reference CPU sample length (0 to skip)")
    ap.add_argument("--sample-temp", type=float, default=1.0, help="temperature of the sampled-decode side figure (0 to skip)")
    ap.add_argument("--prefill", type=int, default=1, help="time the SmolLM2 64-token prefill side figure (0 to skip)")
    ap.add_argument("--probes", action="store_true", help="run only the residency and exchange probes, one JSON line")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run the plain copy kernel once over this many MiB (counter calibration under rocprofv3)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this backend runs one model on one GPU; --gpus {a.gpus} is not a configuration it has "
              "(one GPU's throughput is the figure; multi-GPU sharding is described, not run)", file=sys.stderr)
        sys.exit(2)

    import l3m_amd as A
    if a.probes:
        print(json.dumps({"probes": probes(A)}), flush=True)
        return
    cfg = A.CONFIGS[a.config]
    dtype = a.dtype or cfg.dtype
    with tempfile.TemporaryDirectory() as d:
        path = A.write_model(Path(d) / f"{cfg.name}-{dtype}.l3m", cfg, dtype=dtype, seed=1)
        prompt = A.prompt(1, cfg.vocab, cfg.n_prompt)
        m = A.Model(path)
        log(f"bench: {m.describe()} on {A.lib().l3m_dev_name().decode()}")
        lib = A.lib()
        m.bench_decode(prompt, max(a.warmup, 1))
        lib.l3m_dev_sync()
        w0 = (C.c_double * 3)()
        lib.l3m_decode_work(m._handle(), w0)
        lib.l3m_decode_timer(1, None, None)
        t0 = time.perf_counter()
        m.bench_decode(prompt, a.steps)
        lib.l3m_dev_sync()
        elapsed = time.perf_counter() - t0
        us, launches = C.c_double(), C.c_int()
        lib.l3m_decode_timer(0, C.byref(us), C.byref(launches))
        w1 = (C.c_double * 3)()
        lib.l3m_decode_work(m._handle(), w1)
        value = a.steps / elapsed
        log(f"bench: {a.steps} tokens in {elapsed * 1e3:.2f} ms = {value:.0f} tok/s")
        decode = None
        if m.persistent and launches.value:
            work = [w1[i] - w0[i] for i in range(3)]
            nbytes = decode_bytes(A, m, cfg, work)
            decode = {"kernel": "k_decode", "launches": launches.value, "steps": work[0], "head_steps": work[1],
                      "us": us.value / launches.value, "bytes": nbytes / launches.value, "GBs": nbytes / (us.value * 1e3)}
            log(f"bench: k_decode {launches.value} launches, {work[0]:.0f} steps, {us.value / launches.value:.1f} us per launch, "
                f"{decode['GBs']:.1f} GB/s algorithmic")
        kt = kernel_table(A, m, cfg)
        for r in kt:
            log(f"  {r['kernel']:10s} {r['us']:8.2f} us  {r['GBs']:8.1f} GB/s  x{r['launches_per_token']} = {r['us_per_token']:7.1f} us/token")
        wbytes = A.lib().l3m_weight_bytes(m._handle())
        sampled = sampled_rate(A, m, prompt, a.steps, a.sample_temp) if a.sample_temp > 0 else None
        if sampled:
            log(f"bench: sampled at T={sampled['temperature']}: {sampled['value']} tok/s")
        m.close()
        dom = decode or max(kt, key=lambda r: r["us_per_token"])
        cpu = cpu_baseline(path, prompt, a.cpu_seconds) if a.cpu_seconds > 0 else None
        prefill = prefill_figure(A, d) if a.prefill else None
        if prefill:
            log(f"bench: SmolLM2 q8_0 64-token prompt to first logits: {prefill['ms_prefill']} ms batched, "
                f"{prefill['ms_token_by_token']} ms token by token")
        if cpu:
            log(f"bench: reference CPU {cpu['value']} tok/s on {cpu['cores']} cores")
    matvec = matvec_bench(A, [s for s in a.matvec.split(",") if s]) if a.matvec else None
    if a.copy_mib:
        copy_calibration(A, a.copy_mib << 20)
    pub = PUBLISHED.get((cfg.name, dtype))
    line = {
        "metric": "batch-1 decode tok/s + matvec weight GB/s vs roofline, per dtype",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(elapsed * 1e3 / a.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(value / pub, 3) if pub else None, "dtype": dtype, "data": "synthetic",
        "config": {"workload": f"{cfg.name}-shaped {dtype} Llama, batch-1 greedy decode of {a.steps} tokens from a "
                               f"{cfg.n_prompt}-token seeded prompt, restart at ctx {cfg.ctx}",
                   "dim": cfg.dim, "layers": cfg.n_layers, "heads": cfg.n_heads, "kv_heads": cfg.n_kv_heads,
                   "ffn": cfg.ffn_dim, "vocab": cfg.vocab, "ctx": cfg.ctx, "weights": "random-init N(0,0.02), seed 1"},
        "roofline": {"bound": "hbm", "kernel": dom["kernel"], "achieved": round(dom["GBs"], 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dom["GBs"] / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(cfg.name, dtype, dom["kernel"],
                                                 dom["steps"] / dom["launches"] if "launches" in dom else None),
                     "bytes_per_launch": round(dom["bytes"]), "us_per_launch": round(dom["us"], 3),
                     **({"launches": dom["launches"], "steps": dom["steps"]} if "launches" in dom else {})},
        "step_kernels": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()} for r in kt],
        "weight_bytes_per_token": wbytes,
        "weight_GBs_per_token": round(wbytes * value * 1e-9, 1) if wbytes else None,
        "matvec": matvec,
        "sampled_decode": sampled,
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
