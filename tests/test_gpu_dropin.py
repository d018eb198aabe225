"""The two drop-in boundaries, each through the reference's own code.

The kernel table: fpedd/l3m's library built with its dispatcher able to pick the "hip" table
(oracle/_ref/libl3m_ref_hip.so: dispatch.c with two added lines, linked against libl3m_hip.so). With
L3M_ISA=hip its own l3m_kernels_pick() returns l3m_kernels_hip, whose gemv and attend match its scalar
table on its own packed tiles and prepared vectors (tests/test_kernels.c:71-149 methodology and bars),
and its engine, loaded with L3M_ISA=hip, runs every matvec and attention through the table.

The l3m.h boundary: fpedd/l3m's own CLI (src/main.c, unchanged), linked against
libl3m_hip.so instead of its own library (oracle/Makefile target _ref/l3m-on-hip), runs on the GPU and
passes the reference's own `check` (fast path vs its fp32 reference path: argmax agrees and KL < 0.01
after the prompt, main.c:275-291). Its `generate` prints the same greedy text as the same CLI on the
reference's CPU engine (oracle/_ref/l3m) for a model whose greedy tokens have no near-tie in that range.
Both binaries are built where the reference sources exist and travel with the tree.
"""
import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT
from weights import BF16, F32, MXFP4, Q4_0, Q8_0, rel_err, rows

pytestmark = pytest.mark.gpu
ON_HIP = ROOT / "oracle" / "_ref" / "l3m-on-hip"
ON_CPU = ROOT / "oracle" / "_ref" / "l3m"


def run(binary, *args):
    print(f"dropin: {binary.name} {' '.join(map(str, args))}", flush=True)
    env = {k: v for k, v in os.environ.items() if k != "L3M_ISA"}
    r = subprocess.run([str(binary), *map(str, args)], capture_output=True, timeout=300, env=env)
    print(r.stderr.decode(errors="replace")[-400:], flush=True)
    return r


@pytest.fixture(scope="module")
def cli():
    if not ON_HIP.exists():
        pytest.skip("oracle/_ref/l3m-on-hip was not built (no reference sources where the tree was built)")
    return ON_HIP


@pytest.mark.parametrize("key", [("stories15M", "bf16"), ("stories110M", "q4_0"), ("smollm2", "mxfp4")],
                         ids=lambda k: f"{k[0]}-{k[1]}")
def test_reference_cli_check_passes_on_gpu(cli, models, key):
    path = models.get(*key)
    r = run(cli, "check", path)
    out = r.stdout.decode(errors="replace")
    assert r.returncode == 0, out
    assert "argmax agree" in out and out.strip().endswith("PASS"), out


def test_reference_cli_generate_matches_cpu_engine(cli, models):
    if not ON_CPU.exists():
        pytest.skip("oracle/_ref/l3m missing")
    path = models.get("stories15M", "bf16")
    args = ("generate", path, "-p", "Once upon a time", "-n", "24", "-t", "0")
    gpu, cpu = run(cli, *args), run(ON_CPU, *args)
    assert gpu.returncode == 0 and cpu.returncode == 0
    assert b"(hip)" in gpu.stderr or b"hip" in gpu.stderr
    assert gpu.stdout == cpu.stdout                 # the prompt and 24 greedy tokens, as raw bytes


@pytest.mark.parametrize("extra", [("-t", "0.8", "-s", "7"), ("--ref",), ("--cold",)], ids=["sampled", "ref", "cold"])
def test_reference_cli_generate_options(cli, models, extra):
    """The CLI's `generate` with its other options (main.c:59-75) prints the same text on the GPU library as
    on the reference's CPU engine: temperature sampling with a seed (the same draws from the same logits),
    the fp32 reference path (--ref), and caches emptied before every forward pass (--cold)."""
    if not ON_CPU.exists():
        pytest.skip("oracle/_ref/l3m missing")
    path = models.get("stories15M", "bf16")
    args = ("generate", path, "-p", "Once upon a time", "-n", "24", *extra)
    gpu, cpu = run(cli, *args), run(ON_CPU, *args)
    assert gpu.returncode == 0 and cpu.returncode == 0
    assert gpu.stdout == cpu.stdout


def test_reference_cli_chat_matches_cpu_engine(cli, models):
    """The reference CLI's `chat` (main.c:200-230: the conversation re-fed as text each turn) with two turns
    piped in: the GPU library prints the same greedy replies as the same CLI on the reference's CPU engine."""
    if not ON_CPU.exists():
        pytest.skip("oracle/_ref/l3m missing")
    path = models.get("stories15M", "bf16")
    env = {k: v for k, v in os.environ.items() if k != "L3M_ISA"}
    outs = []
    for binary in (cli, ON_CPU):
        r = subprocess.run([str(binary), "chat", str(path), "-n", "16", "-t", "0"], input=b"Once upon a time\nThe cat sat\n",
                           capture_output=True, timeout=300, env=env)
        print(r.stderr.decode(errors="replace")[-300:], flush=True)
        assert r.returncode == 0
        outs.append(r.stdout)
    assert outs[0] == outs[1]
    assert outs[0].count(b"> ") == 3                  # two turns answered, then the prompt for a third


def test_reference_cli_bench_on_gpu(cli, models):
    """The reference CLI's `bench` (main.c:233-263) on the GPU library: its perf line for one model (the
    description ends in "(hip)", then tok/s, us/tok and the compute/wait split of l3m_perf), and its
    markdown table for two models, one row each."""
    import re
    a, b = models.get("stories110M", "q4_0"), models.get("stories15M", "bf16")
    r = run(cli, "bench", a, "-n", "64")
    out = r.stdout.decode(errors="replace")
    assert r.returncode == 0, out
    assert "(hip)" in out, out
    m = re.search(r"([0-9]+) tok/s\s+([0-9.]+) us/tok\s+\(compute ([0-9.]+), wait ([0-9.]+)\)", out)
    assert m, out
    tok_s, us, compute, wait = (float(g) for g in m.groups())
    assert tok_s > 1000 and abs(compute + wait - us) < 0.2 * us, out
    r = run(cli, "bench", "--md", a, b, "-n", "32")
    out = r.stdout.decode(errors="replace")
    assert r.returncode == 0, out
    rows = [line for line in out.splitlines() if line.startswith("| ") and "(hip)" in line]
    assert len(rows) == 2, out


TOL = {F32: 1e-3, BF16: 1e-3, Q8_0: 1e-3, Q4_0: 5e-3, MXFP4: 5e-3}


@pytest.fixture(scope="module")
def ref_hip(monkeypatch_module):
    from oracle.oracle import Reference
    if not Reference.available(Reference.HIP_PATH):
        pytest.skip("oracle/_ref/libl3m_ref_hip.so was not built (no reference sources where the tree was built)")
    monkeypatch_module.setenv("L3M_ISA", "hip")
    return Reference(Reference.HIP_PATH)


@pytest.fixture(scope="module")
def monkeypatch_module():
    mp = pytest.MonkeyPatch()
    yield mp
    mp.undo()


def test_reference_dispatcher_picks_hip_table(ref_hip):
    import l3m_amd as A
    from oracle.oracle import _Table
    name, addr = ref_hip.pick()
    print(f"dispatcher: L3M_ISA=hip picked {name}", flush=True)
    hip = _Table.in_dll(A.lib(), "l3m_kernels_hip")
    assert name == "hip" and addr == C.addressof(hip)
    assert ref_hip.lib.l3m_kernels_usable(C.addressof(hip)) == 1
    assert ref_hip.usable("scalar")                   # the CPU tables stay as they were


@pytest.mark.parametrize("dtype", [F32, BF16, Q8_0, Q4_0, MXFP4], ids=["f32", "bf16", "q8_0", "q4_0", "mxfp4"])
def test_picked_table_matches_scalar_table(ref_hip, dtype):
    """gemv through the table the reference's dispatcher picked, on tiles its l3m_pack_tile packed and the
    vector its l3m_vec_prepare prepared, against its scalar table (test_kernels.c:71-122)."""
    from oracle.oracle import _Table
    table = _Table.from_address(ref_hip.pick()[1])
    for k, ntiles in [(288, 3), (768, 2), (2048, 4)]:
        n = ntiles * 16
        w = rows(dtype, n, k, seed=3 * k + dtype)
        tiles = ref_hip.pack_tiles(dtype, [w[i] if i < n - 2 else None for i in range(n)], k)
        x = np.random.default_rng(k + 1).standard_normal(k).astype(np.float32)
        v, keep = ref_hip.prepare(dtype, x)
        y = np.zeros(n, np.float32)
        table.gemv[dtype](y.ctypes.data_as(C.POINTER(C.c_float)), tiles.ctypes.data, ntiles, k, C.byref(v))
        want = ref_hip.gemv("scalar", dtype, tiles, ntiles, k, x)
        print(f"dispatcher: gemv dtype {dtype} k {k}: rel err {rel_err(y, want):.2e}", flush=True)
        assert rel_err(y, want) < TOL[dtype], (k, rel_err(y, want))
    rng = np.random.default_rng(dtype)
    hd, pos, stride = 64, 77, 192
    q = rng.standard_normal(hd).astype(np.float32)
    kk = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBFFF
    vv = rng.integers(0, 1 << 16, (pos + 1) * stride, dtype=np.uint16) & 0xBFFF
    out = np.zeros(hd, np.float32)
    f, u16 = C.POINTER(C.c_float), C.POINTER(C.c_uint16)
    table.attend(out.ctypes.data_as(f), q.ctypes.data_as(f), kk.ctypes.data_as(u16), vv.ctypes.data_as(u16), pos, hd, stride)
    assert np.abs(out - ref_hip.attend("scalar", q, kk, vv, pos, hd, stride)).max() <= 1e-5


def test_reference_engine_runs_on_picked_table(ref_hip, models, monkeypatch_module):
    """The reference's engine loaded with L3M_ISA=hip describes itself as (hip) and generates through the
    table; its logits after the prompt and its greedy tokens agree with the same engine on its scalar
    table (max |logit difference| within 1e-3 of max |logit|, the matvec bar)."""
    import l3m_amd as A
    cfg = A.Config("dispatch", dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn_dim=128, vocab=320, ctx=64, dtype="q8_0")
    path = models.get(cfg)
    prompt = A.prompt(5, cfg.vocab, 4)
    on_hip = ref_hip.load(path, cpus=[0, 1])
    assert on_hip.describe().endswith("(hip)"), on_hip.describe()
    got = on_hip.generate(prompt, 12)
    lg = on_hip.logits()
    monkeypatch_module.setenv("L3M_ISA", "scalar")
    try:
        on_cpu = ref_hip.load(path, cpus=[0, 1])
        assert on_cpu.describe().endswith("(scalar)"), on_cpu.describe()
        want = on_cpu.generate(prompt, 12)
        lw = on_cpu.logits()
    finally:
        monkeypatch_module.setenv("L3M_ISA", "hip")
    err = float(np.abs(lg - lw).max() / np.abs(lw).max())
    print(f"dispatcher: engine on hip {got}\ndispatcher: engine on scalar {want}\nlogit rel err {err:.2e}", flush=True)
    assert err < 1e-3
    assert got == want
