"""Benchmark of the Backend_hip hot path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]``

The default workload is the configuration BASELINE.json's metric is quoted
on, config 2 (row ops): reduce_rows(add), reduce_rows(max) and
scan_rows(add) over an f32 [8192; 8192] matrix, plus an inclusive scan of
an i32 vector of 2^28 elements. One step is one run of both compiled
programs over inputs already resident in HBM (run_resident_into, outputs
preallocated, no host traffic). ``value`` is HBM bytes per second over
the K timed steps: the bytes the step's kernels read and write of
materialised tensors, each tensor a kernel reads counted once
(``config.moved_bytes_per_step``; scratch excluded). It is checked
against the 8 TB/s peak before the line is printed. The fusion plan's own
algorithmic total (each root's inputs read once and output written once,
counting reads the lowering removed: the read of r by config 1's s = sum r,
folded inside r's map; the second and third reads of x by config 2's
sibling row roots, fused into one kernel) is
``config.plan_bytes_per_step``, and its rate ``config.plan_gbs``.
Other configs (``--config saxpy``,
``chain``, ``scatter``, ``scatter_perm``, ``matmul``, ``matmul64``, ``matmul_grad``,
``mc``, ``mc64``, ``mc_greeks``) print their own line in the same format;
``saxpy_hbm`` and ``chain_hbm`` run config 1's graphs over 2^28 elements,
whose inputs cannot stay in the 256 MB MALL between steps (config 1's
2^24 ones do), for the map template's HBM-only rate.
``poly`` and ``poly64`` are the reference benchmark's own workload
(bench/bench.ml): the degree-64 Horner chain plus its sum over 2^24
elements; their ``value`` is GFLOP/s with the input resident, and their
``whole_run`` carries the reference's RESULT fields (saxpy and poly whole
runs, best of 5, and the host-device copy rates) beside its published
A100 figures; ``--pinned`` runs them from page-locked host memory, as the
reference's own flag does.
``bs``, ``bs_greeks`` (and their f64 ``bs64``, ``bs_greeks64``) are the
reference's S20 timing row: the one-step Black-Scholes price and its
Greeks adjoint at 2^22 paths; their ``whole_run`` is timed as S20 times it
and set against the published A100 figure.

The JSON line also carries ``roofline`` for the dominant kernel (its
algorithmic bytes or flops per launch over its mean launch time, timed with
HIP events on the executor's stream inside the timed region) and
``cpu_baseline``: the CPU oracle (a C restatement of the reference
interpreter, single-threaded) timed on a bounded sample of the same
workload on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP32_MFMA_TFLOPS = 157.3
FP64_MFMA_TFLOPS = 78.6


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def plan_bytes(H, graph):
    """Per kernel of the plan, as the code generator attributes them:
    (template, root bytes, moved bytes). Root bytes are the fusion plan's
    algorithmic bytes of the root the kernel computes: each element the
    root reads counted once (a gather one element per output, a broadcast
    source one), its output written once. Moved bytes are what the kernel
    itself reads and writes of materialised tensors, each tensor read once:
    the root bytes, less reads the lowering removed (a reduction folded
    inside the map that writes its input reads nothing back; row roots over
    one input fused into one kernel read it once). Helper kernels carry 0."""
    out = {}
    for line in H.plan(graph).splitlines():
        f = line.split()
        if f[0] == "kernel":
            out[f[1]] = (f[2], int(f[f.index("bytes") + 1]), int(f[f.index("moved") + 1]))
    return out


class Workload:
    def __init__(self, name, programs, unit, dtype, describe):
        self.name = name
        self.programs = programs  # list of (graph, compiled, inputs residents, output residents)
        self.unit = unit
        self.dtype = dtype
        self.describe = describe


def device_inputs(H, gen_graph, seed):
    import numpy as np

    c = H.compile(gen_graph)
    seed_r = H.upload(np.array(seed, dtype=np.int32))
    out = H.run_resident(c, [("seed", seed_r)])
    H.free_resident(seed_r)
    c.release()
    return out[0][1]


def alloc_outputs(H, c):
    from cudacaml_amd.runtime import Buffer

    return [(o.name, H.Resident(Buffer.alloc(o.nbytes), o.dtype, o.shape)) for o in c.outputs]


def build_workload(name, H, C):
    """Compile the programs of one config and put its inputs in HBM."""
    from cudacaml_amd.examples import black_scholes as bs
    from cudacaml_amd.ir import F32, F64

    progs = []

    def add(g, inputs):
        c = H.compile(g)
        progs.append((g, c, inputs, alloc_outputs(H, c)))

    if name == "rows":
        x = device_inputs(H, C.gen_uniform_pm1((C.ROWS2, C.ROWS2)), 3)
        v = device_inputs(H, C.gen_small_ints((C.SCAN2,)), 4)
        add(C.rows(), [("x", x)])
        add(C.global_scan(), [("v", v)])
        return Workload(name, progs, "GB/s", "f32/i32",
                        "config2: reduce_rows add+max and scan_rows add over f32[8192,8192]; "
                        "inclusive scan over i32[2^28]")
    if name == "copy":
        # calibration: one plain copy kernel of known size (1 GiB read, 1 GiB written)
        from cudacaml_amd import dsl as Dsl
        from cudacaml_amd.ir import Graph

        x = device_inputs(H, C.gen_uniform_pm1((1 << 28,)), 1)
        add(Graph.create("copy", [("r", Dsl.map(lambda e: e, Dsl.param("x", F32, (1 << 28,))))]), [("x", x)])
        return Workload(name, progs, "GB/s", "f32", "calibration: copy of f32[2^28]")
    if name in ("saxpy", "chain", "saxpy_hbm", "chain_hbm"):
        # the _hbm variants: the same graphs over 2^28 elements, whose 1-2
        # GiB inputs cannot stay in the 256 MB MALL between steps
        n = (1 << 28) if name.endswith("_hbm") else C.N1
        what = "2^28 (beyond the MALL)" if name.endswith("_hbm") else "2^24"
        x = device_inputs(H, C.gen_uniform_pm1((n,)), 1)
        if name.startswith("saxpy"):
            y = device_inputs(H, C.gen_uniform_pm1((n,)), 2)
            add(C.saxpy(n), [("x", x), ("y", y)])
            desc = ("config1: saxpy r=2x+y, s=sum r over f32[%s]; s is folded inside r's map kernel, so "
                    "r is never read back" % what)
        else:
            add(C.chain(n), [("x", x)])
            desc = "config1b: 5-map chain over f32[%s], one fused kernel" % what
        return Workload(name, progs, "GB/s", "f32", desc)
    if name in ("scatter", "scatter_perm"):
        src = device_inputs(H, C.gen_uniform_pm1((C.N3,)), 5)
        if name == "scatter":
            idx = device_inputs(H, C.gen_bin_indices(C.N3, 20), 6)
            add(C.scatter_gather(), [("idx", idx), ("src", src)])
            desc = "config3: scatter_add of f32[2^26] into 2^20 bins (uniform idx) + gather back"
        else:
            import numpy as np

            perm = H.upload(C.permutation(7, C.N3))
            add(C.scatter_gather(C.N3, C.N3), [("idx", perm), ("src", src)])
            desc = "config3b: scatter_add of f32[2^26] through a permutation into 2^26 bins + gather back"
            del np
        return Workload(name, progs, "GB/s", "f32", desc)
    if name in ("matmul", "matmul64", "matmul_grad"):
        dt = F64 if name == "matmul64" else F32
        n = C.MM_F64 if name == "matmul64" else C.MM_F32
        a = device_inputs(H, C.gen_normals((n, n), dt), 8)
        b = device_inputs(H, C.gen_normals((n, n), dt), 9)
        g = C.matmul_grad(n, dt) if name == "matmul_grad" else C.matmul(n, dt)
        add(g, [("a", a), ("b", b)])
        return Workload(name, progs, "TFLOP/s", dt.name, "config4: %s %s %dx%d" % (name, dt.name, n, n))
    if name in ("mc", "mc64", "mc_greeks"):
        dt = F64 if name == "mc64" else F32
        g = C.mc_greeks() if name == "mc_greeks" else C.mc_paths(C.PATHS5, C.STEPS5, dt)
        ins = [(k, H.upload(v)) for k, v in bs.inputs(dt, seed=7)]
        add(g, ins)
        desc = "config5: BS MC %s 2^22 paths x 64 steps %s" % ("greeks" if name == "mc_greeks" else "price", dt.name)
        if dt is F32:
            desc += ("; at seed 7 about 12 of the 2^28 f32 draws are +-inf under the reference's own f32 generator "
                     "(rng.ml:61-71: u rounds to 1.0 in f32), so the price is +inf and the Greeks NaN, "
                     "as the interpreter gives them")
        return Workload(name, progs, "paths/s", dt.name, desc)
    if name in ("poly", "poly64"):
        from cudacaml_amd.examples import refbench as RB

        dt = F64 if name == "poly64" else F32
        x = H.upload(RB.x_input(RB.N, dt))
        add(RB.poly_graph(RB.N, dt), [("x", x)])
        return Workload(name, progs, "GFLOP/s", dt.name,
                        "the reference benchmark's poly: degree-64 Horner chain (63 fused maps) + sum over "
                        "%s[2^24], x[i] = (i mod 17) - 8, c[j] = 1/(j+1) (bench/bench.ml:97-111,223,253)" % dt.name)
    if name in BS_CONFIGS:
        dt = F64 if name.endswith("64") else F32
        greeks = name.startswith("bs_greeks")
        g = bs.call_greeks(C.PATHS5, dt) if greeks else bs.call_mc(C.PATHS5, dt)
        ins = [(k, H.upload(v)) for k, v in bs.inputs(dt, seed=1)]
        add(g, ins)
        return Workload(name, progs, "paths/s", dt.name,
                        "BS MC %s, one step, 2^22 paths %s (the reference's S20 timing row)"
                        % ("Greeks adjoint (delta, vega, rho)" if greeks else "price", dt.name))
    raise SystemExit("unknown config %s" % name)


# The reference's published S20 row (README.md:152-157): Backend_cuda.run of
# Bs.call_mc / Bs.call_greeks at 2^22 paths, f32, on an A100-SXM4-40GB,
# mean of 5 warm runs, host inputs to host outputs.
BS_CONFIGS = ("bs", "bs64", "bs_greeks", "bs_greeks64")
BS_PUBLISHED_MS = {"bs": 0.2, "bs_greeks": 0.7}


# The reference's published host-transfer rates on the A100: a 64 MiB
# round trip, pinned against pageable (README.md:198-201, S18).
PUBLISHED_A100_COPY_GBS = {"pinned": 12.3, "pageable": 4.8}


def refbench_whole_runs(H, dt, reps=5, pinned=False):
    """The reference benchmark's RESULT fields (bench/bench.ml:227-300),
    measured as it measures them: best of ``reps`` whole runs (upload,
    launches, download) of saxpy and poly after one warm run, and the
    2^24-element host-to-device and device-to-host copy rates. With
    ``pinned`` (the reference's --pinned, bench/bench.ml:126-145) the
    inputs and the copy sink are page-locked host memory (Pinned.alloc),
    so the copies DMA straight from and into them; the run's outputs are
    fresh host values either way, as Backend.run returns them."""
    import numpy as np

    from cudacaml_amd.examples import refbench as RB
    from cudacaml_amd.runtime import Buffer, Pinned

    def best(f):
        t = math.inf
        for _ in range(reps):
            t0 = time.perf_counter()
            f()
            t = min(t, time.perf_counter() - t0)
        return t

    n = RB.N
    x, y = RB.x_input(n, dt), RB.y_input(n, dt)
    sink = np.empty_like(x)
    if pinned:
        x, y = Pinned.of_value(x), Pinned.of_value(y)
        sink = Pinned.alloc(dt, x.shape)
        assert Pinned.is_pinned(x) and Pinned.is_pinned(y) and Pinned.is_pinned(sink)
    buf = Buffer.alloc(x.nbytes)
    buf.upload(x)
    t_h2d = best(lambda: buf.upload(x))
    t_d2h = best(lambda: buf.download(sink))
    buf.free()
    cs = H.compile(RB.saxpy_graph(n, dt))
    H.run(cs, [("x", x), ("y", y)])
    t_saxpy = best(lambda: H.run(cs, [("x", x), ("y", y)]))
    cs.release()
    cp = H.compile(RB.poly_graph(n, dt))
    H.run(cp, [("x", x)])
    t_poly = best(lambda: H.run(cp, [("x", x)]))
    cp.release()
    return {"saxpy_cuda_s": round(t_saxpy, 5), "poly_cuda_s": round(t_poly, 5),
            "poly_gflops": round(n * RB.poly_flops() / t_poly / 1e9, 2),
            "h2d_gbs": round(x.nbytes / t_h2d / 1e9, 2), "d2h_gbs": round(x.nbytes / t_d2h / 1e9, 2),
            "hostmem": "pinned" if pinned else "pageable", "n": n, "reps": reps,
            "published_a100_copy_gbs": {"value": PUBLISHED_A100_COPY_GBS["pinned" if pinned else "pageable"],
                                        "what": "64 MiB host transfer on the A100, README.md:198-201"}}


def step(H, w, sync=False):
    for g, c, ins, outs in w.programs:
        H.run_resident_into(c, ins, outs, sync=sync)


def host_cpu():
    """The host's CPU model and the cores this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"model": model, "nproc": os.cpu_count(), "usable": usable}


def cpu_baseline(name, C, H, w):
    """The oracle (one thread) on the whole workload or a bounded sample of
    it, over the benchmark's own inputs (downloaded from the device, or the
    leading part of the same generator stream). Returns (value in the
    config's unit, unit, sample description, seconds)."""
    import numpy as np

    import oracle
    from cudacaml_amd.examples import black_scholes as bs
    from cudacaml_amd.ir import F32, F64

    def timed(g, ins):
        c = oracle.Interp.compile(g)
        t0 = time.perf_counter()
        oracle.Interp.run(c, ins)
        return time.perf_counter() - t0

    def host_inputs(k=0):
        return [(n, H.download(r)) for n, r in w.programs[k][2]]

    def plan_total(g):
        return sum(b for _, (_, b, _) in plan_bytes(H, g).items())

    if name in ("poly", "poly64"):
        from cudacaml_amd.examples import refbench as RB

        dt = F64 if name == "poly64" else F32
        n = 1 << 22
        secs = timed(RB.poly_graph(n, dt), [("x", RB.x_input(n, dt))])
        return (n * RB.poly_flops() / secs / 1e9, "GFLOP/s",
                "poly graph on the first 2^22 of the 2^24 elements (a quarter of the workload)", secs)
    if name == "rows":
        x, v = host_inputs(0)[0][1], host_inputs(1)[0][1]
        secs = timed(C.rows(), [("x", x)]) + timed(C.global_scan(), [("v", v)])
        nbytes = plan_total(C.rows()) + plan_total(C.global_scan())
        return nbytes / secs / 1e9, "GB/s", "the whole workload: rows graph on f32[8192,8192] + global scan on i32[2^28]", secs
    if name in ("saxpy_hbm", "chain_hbm"):
        # the oracle's rate does not depend on the length: time the 2^24
        # graph on the leading 2^24 elements of the same inputs
        n = C.N1
        g = C.saxpy(n) if name.startswith("saxpy") else C.chain(n)
        ins = [(k, v[:n]) for k, v in host_inputs(0)]
        secs = timed(g, ins)
        return plan_total(g) / secs / 1e9, "GB/s", "the graph on the first 2^24 of the 2^28 elements", secs
    if name in ("saxpy", "chain", "scatter", "scatter_perm"):
        g, ins = w.programs[0][0], host_inputs(0)
        secs = timed(g, ins)
        return plan_total(g) / secs / 1e9, "GB/s", "the whole workload", secs
    if name in ("matmul", "matmul64", "matmul_grad"):
        # The interpreter's matmul is one sequential k-loop per output
        # (R9), so its rate is the same for every row: time the leading
        # rows of the benchmark's own product and report that rate.
        ins = dict(host_inputs(0))
        a, b = ins["a"], ins["b"]
        n = b.shape[1]
        rows = 64 if a.dtype == np.float64 else 32
        dt = F64 if a.dtype == np.float64 else F32
        secs = timed(C.matmul(n, dt, k=a.shape[1], m=rows), [("a", np.ascontiguousarray(a[:rows])), ("b", b)])
        what = "the first %d rows of A@B (%s %dx%d), %.2f%% of the product's flops" % (
            rows, dt.name, n, n, 100.0 * rows / a.shape[0])
        if name == "matmul_grad":
            what += "; the rate applies to the grad graph's three %d^3 products (extrapolated)" % n
        return 2 * rows * a.shape[1] * n / secs / 1e12, "TFLOP/s", what, secs
    if name in ("mc", "mc64", "mc_greeks"):
        # Draw counters are flat indices (path * steps + step), so the
        # first P paths of the workload see exactly the same draws.
        dt = F64 if name == "mc64" else F32
        p = 1 << 14
        g = C.mc_greeks(p, C.STEPS5, dt) if name == "mc_greeks" else C.mc_paths(p, C.STEPS5, dt)
        secs = timed(g, bs.inputs(dt, seed=7))
        return p / secs, "paths/s", "the first 2^14 of the 2^22 paths (same draws), 64 steps", secs
    if name in BS_CONFIGS:
        dt = F64 if name.endswith("64") else F32
        p = 1 << 20
        g = bs.call_greeks(p, dt) if name.startswith("bs_greeks") else bs.call_mc(p, dt)
        secs = timed(g, bs.inputs(dt, seed=1))
        return p / secs, "paths/s", "the first 2^20 of the 2^22 paths (same draws)", secs
    raise SystemExit("no CPU baseline for %s" % name)


def pmc_child(args):
    """Child of a counter pass: the workload's warm-up and steps, then the
    copy calibration kernel; prints the calibration kernel's name as JSON."""
    from cudacaml_amd import backend_hip as H
    from cudacaml_amd.examples import configs as C

    w = build_workload(args.config, H, C)
    cal = build_workload("copy", H, C)
    copy_name = list(plan_bytes(H, cal.programs[0][0]))[0]
    for _ in range(2 + args.steps):
        step(H, w)
    for _ in range(2):
        step(H, cal)
    from cudacaml_amd.runtime import Device

    Device.synchronize()
    print(json.dumps({"copy": copy_name}), flush=True)


COPY_BYTES = (1 << 28) * 4  # read once and written once by the calibration kernel


# Configs whose dominant kernel is bound by instruction issue rather than
# HBM: two more counter passes. A SIMD issues one wave64 VALU instruction a
# quad-cycle (4 clocks), and gfx950 issues a second one in the same
# quad-cycle where the pair allows it (SQ_ACTIVE_INST_VALU2 counts those
# quad-cycles). SQ_ACTIVE_INST_VALU counts the quad-cycles of each VALU
# instruction, so the quad-cycles in which a SIMD issues VALU work at all
# are ACTIVE_INST_VALU - ACTIVE_INST_VALU2; over the dispatch's SIMD
# quad-cycles that is the share of the issue ceiling the kernel uses (1.0:
# a VALU instruction issued every quad-cycle on every SIMD). The second
# pass splits the VALU instructions by class. Packed FP32 is off in every
# build here, so it is not counted.
VALU_CONFIGS = ("poly", "poly64", "mc", "mc64", "mc_greeks", "bs", "bs64", "bs_greeks", "bs_greeks64")
VALU_CLASSES = ("SQ_INSTS_VALU_INT32", "SQ_INSTS_VALU_INT64", "SQ_INSTS_VALU_FMA_F32", "SQ_INSTS_VALU_FMA_F64",
                "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_VALU_TRANS_F64", "SQ_INSTS_VALU_CVT", "SQ_INSTS_VALU_ADD_F64")


# Matmul configs: one more counter pass for the matrix cores.
MFMA_CONFIGS = ("matmul", "matmul64", "matmul_grad")
# GRBM_GUI_ACTIVE is counted per XCC and the csv sums the 8 of them; a
# dispatch that covers every XCC runs for (sum / 8) cycles.
XCC_COUNT = 8
SIMDS_PER_CU = 4
# Published MI355X matrix peaks at the 2.4 GHz they are quoted for, as
# flops per clock for the whole chip.
MFMA_CLOCK_HZ = 2.4e9


def counter_passes(config):
    """The rocprofv3 --pmc passes for a config, each a list of counters
    collected together: the two traffic counters, then the VALU
    instructions with the same dispatches' cycle count (issue-bound
    configs), or the matrix-core busy cycles and math operations with the
    cycle count (matmul configs)."""
    passes = [["FETCH_SIZE"], ["WRITE_SIZE"]]
    if config in VALU_CONFIGS:
        passes.append(["SQ_INSTS_VALU", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_VALU2", "GRBM_GUI_ACTIVE"])
        passes.append(list(VALU_CLASSES) + ["GRBM_GUI_ACTIVE"])
    if config in MFMA_CONFIGS:
        passes.append(["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_VALU_MFMA_MOPS_F64",
                       "GRBM_GUI_ACTIVE"])
    return passes


def measure_counters(config, steps=2):
    """rocprofv3 counter passes over the workload (counter_passes), each
    run as a child process before this process touches the GPU. Values are
    per dispatch (the csv's sum over the counter's instances). Returns
    ({kernel: {counter: median}}, copy kernel name) or (None, reason)."""
    import csv
    import glob
    import shutil
    import statistics
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    per = {}
    copy_name = None
    for group in counter_passes(config):
        out = tempfile.mkdtemp(prefix="cchip_pmc_", dir="/tmp")
        cmd = [exe, "--pmc"] + group + ["--output-format", "csv", "-d", out, "-o", "p", "--",
                                         sys.executable, os.path.abspath(__file__), "--config", config, "--steps",
                                         str(steps), "--pmc-child"]
        env = dict(os.environ, TMPDIR="/tmp")
        log("counters: %s pass" % " ".join(group))
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                               timeout=180, start_new_session=True)
        except subprocess.TimeoutExpired:
            return None, "rocprofv3 %s pass timed out" % " ".join(group)
        lines = [l for l in r.stdout.decode(errors="replace").splitlines() if l.startswith("{")]
        if r.returncode != 0 or not lines:
            return None, "rocprofv3 %s pass failed (rc %d)" % (" ".join(group), r.returncode)
        copy_name = json.loads(lines[-1])["copy"]
        files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            return None, "no counter file from the %s pass" % " ".join(group)
        vals = {}
        with open(files[0]) as f:
            for i, row in enumerate(csv.DictReader(f)):
                if row["Counter_Name"] not in group:
                    continue
                # rows of one dispatch (one per counter instance, if the
                # csv splits them) are summed
                d = row.get("Dispatch_Id") or row.get("Correlation_Id") or str(i)
                by = vals.setdefault((row["Kernel_Name"], row["Counter_Name"]), {})
                by[d] = by.get(d, 0.0) + float(row["Counter_Value"])
        shutil.rmtree(out, ignore_errors=True)
        for (k, cn), by_dispatch in vals.items():
            per.setdefault(k, {})[cn] = statistics.median(by_dispatch.values())
    return per, copy_name


def traffic_of(counters, kernel):
    """HBM bytes per launch of ``kernel``: each counter scaled by what the
    same counter reads for a plain copy kernel of known size. Returns
    (traffic_bytes, detail) or (None, reason)."""
    per, copy_name = counters
    if per is None:
        return None, copy_name
    dom, cal = per.get(kernel, {}), per.get(copy_name, {})
    if len(dom) < 2 or len(cal) < 2:
        return None, "kernel rows missing from the counter passes"
    fetch_scale = COPY_BYTES / (cal["FETCH_SIZE"] * 1024)
    write_scale = COPY_BYTES / (cal["WRITE_SIZE"] * 1024)
    fetch = dom["FETCH_SIZE"] * 1024 * fetch_scale
    write = dom["WRITE_SIZE"] * 1024 * write_scale
    detail = {"kernel": kernel, "fetch_kib": dom["FETCH_SIZE"], "write_kib": dom["WRITE_SIZE"],
              "fetch_scale": round(fetch_scale, 4), "write_scale": round(write_scale, 4),
              "fetch_bytes": int(fetch), "write_bytes": int(write)}
    return int(fetch + write), detail


def kernel_elements(H, w, kernel):
    """Elements a kernel processes: its largest argument that is not the
    error word or scratch (the output of a map or scan, the input of a
    reduction)."""
    for g, _, _, _ in w.programs:
        sizes = {}
        for line in H.plan(g).splitlines():
            f = line.split()
            if f[0] == "buffer" and f[-1] not in ("err", "scratch"):
                sizes[f[1]] = int(f[4])
            elif f[0] == "kernel" and f[1] == kernel:
                outs = [sizes[a] for a in f[f.index("args") + 1:] if a in sizes]
                return max(outs) if outs else 0
    return 0


def kernel_table(H, w):
    """{kernel: (template, moved bytes, compiled, root bytes)} over the
    workload's programs."""
    kinfo = {}
    for g, c, _, _ in w.programs:
        for k, (role, b, m) in plan_bytes(H, g).items():
            kinfo[k] = (role, m, c, b)
    return kinfo


def dominant(H, w, config, timed=True):
    """Of the kernels that move a root's bytes, the one that takes the most
    time per step (one timed step per kernel, HIP events around its
    launches), or, without timing, the one with the most bytes (the matmul
    for matmul configs): (name, role, moved bytes, compiled, root bytes,
    table). Helper kernels (a scatter's counts and accumulate, a split
    reduction's fold) carry no bytes of their own, so no roofline can be put
    on them; the profiles list their times."""
    kinfo = kernel_table(H, w)
    if timed:
        from cudacaml_amd.runtime import Device

        best, best_ms = None, -1.0
        for k, (role, b, c, _) in kinfo.items():
            if b <= 0:
                continue
            H.time_kernel(c, k)
            step(H, w)
            Device.synchronize()
            each = H.timing_each(c)
            H.time_kernel(c, None)
            ms = sum(each)
            if ms > best_ms:
                best, best_ms = k, ms
        dom = best
    else:
        dom = max(kinfo.items(), key=lambda kv: kv[1][1])[0]
        if config.startswith("matmul"):
            dom = [k for k, v in kinfo.items() if v[0].startswith("matmul")][0]
    return (dom,) + kinfo[dom] + (kinfo,)


def whole_run_ms(H, w, reps=3, mean=False):
    """Time of a synchronous run from host arrays: upload, launches,
    download (pageable host memory, as Executor.run); the median of
    ``reps`` runs, or after one warm run their mean (the reference's S20
    timing, test_system.ml:225-245)."""
    import statistics

    hosts = [(c, [(n, H.download(r)) for n, r in ins]) for _, c, ins, _ in w.programs]
    if mean:
        for c, ins in hosts:
            H.run(c, ins)
        t0 = time.perf_counter()
        for _ in range(reps):
            for c, ins in hosts:
                H.run(c, ins)
        return (time.perf_counter() - t0) * 1e3 / reps
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for c, ins in hosts:
            H.run(c, ins)
        ts.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(ts)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="rows")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--no-whole-run", action="store_true", help="skip the host-to-host run timing")
    ap.add_argument("--pinned", action="store_true",
                    help="poly/poly64: page-locked host memory for the whole runs (the reference's --pinned)")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this backend runs on one GPU; multi-GPU runs (Multi) are out of scope. Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.pmc_child:
        pmc_child(args)
        return
    # Counter passes first: they are child processes, started before this
    # process initialises the GPU.
    counters = (None, "skipped (--no-traffic)")
    if not args.no_traffic:
        counters = measure_counters(args.config)

    import statistics

    from cudacaml_amd import backend_hip as H
    from cudacaml_amd.examples import configs as C
    from cudacaml_amd.runtime import Device

    if not Device.available():
        raise SystemExit("bench.py: no HIP device")
    info = Device.info()
    log("device: %s %s, %d CUs" % (info.name, info.arch, info.multiprocessors))
    t0 = time.perf_counter()
    w = build_workload(args.config, H, C)
    log("compiled and generated inputs in %.1fs" % (time.perf_counter() - t0))

    for _ in range(args.warmup):
        step(H, w)
    Device.synchronize()
    dom, dom_role, dom_bytes, dom_c, dom_root_bytes, kinfo = dominant(H, w, args.config)
    traffic, traffic_detail = traffic_of(counters, dom)
    log("traffic:", traffic, traffic_detail)
    Device.synchronize()
    H.time_kernel(dom_c, dom)
    Device.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(H, w)
    Device.synchronize()
    elapsed = time.perf_counter() - t0
    each = H.timing_each(dom_c)
    H.time_kernel(dom_c, None)
    step(H, w, sync=True)  # surfaces any device-side error of the timed runs

    ms_per_step = elapsed * 1e3 / args.steps
    plan_total = sum(rb for _, (_, _, _, rb) in kinfo.items())
    moved_total = sum(m for _, (_, m, _, _) in kinfo.items())
    if w.unit == "GB/s":
        # HBM bytes the step's kernels read and write (inputs resident)
        value = moved_total * args.steps / elapsed / 1e9
        if value > HBM_PEAK_GBS:
            raise SystemExit("bench.py: %.1f GB/s is above the %.0f GB/s HBM peak: the moved bytes of %s "
                             "overcount what its kernels read and write" % (value, HBM_PEAK_GBS, args.config))
    elif w.unit == "TFLOP/s":
        flops = 0
        for g, c, _, _ in w.programs:
            for t in g.order:
                if t.kind == "matmul":
                    flops += 2 * t.shape[0] * t.shape[1] * t.a.shape[1]
        value = flops * args.steps / elapsed / 1e12
    elif w.unit == "GFLOP/s":
        from cudacaml_amd.examples import refbench as RB

        value = RB.N * RB.poly_flops() * args.steps / elapsed / 1e9
    else:
        value = C.PATHS5 * args.steps / elapsed
    dom_avg_ms = sum(each) / max(1, len(each))
    if dom_role.startswith("matmul"):
        uid = int(dom.split("_")[1])
        mm = [t for g, _, _, _ in w.programs for t in g.order if t.uid == uid][0]
        fl = 2 * mm.shape[0] * mm.shape[1] * mm.a.shape[1]
        peak = FP64_MFMA_TFLOPS if mm.dtype.name == "f64" else FP32_MFMA_TFLOPS
        achieved = fl / (dom_avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "traffic": traffic, "flops_per_launch": fl}
    else:
        achieved = dom_bytes / (dom_avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}
    per = counters[0] or {}
    simds = info.multiprocessors * SIMDS_PER_CU
    dc = per.get(dom, {})
    if (args.config in VALU_CONFIGS and "SQ_ACTIVE_INST_VALU" in dc and "SQ_ACTIVE_INST_VALU2" in dc
            and dc.get("GRBM_GUI_ACTIVE")):
        # Issue-bound kernels: the quad-cycles in which each SIMD issued VALU
        # work (ACTIVE_INST_VALU less the quad-cycles that issued two) over
        # the dispatch's SIMD quad-cycles (GRBM_GUI_ACTIVE of the same
        # pass), so no clock rate is assumed; also the wave64 instructions,
        # lane-instructions per element of the kernel's output, the share of
        # VALU quad-cycles that issued two, the instructions by class, and
        # the clock those cycles imply over this run's HIP-event time.
        winst = dc.get("SQ_INSTS_VALU", 0.0)
        active, dual = dc["SQ_ACTIVE_INST_VALU"], dc["SQ_ACTIVE_INST_VALU2"]
        cycles = dc["GRBM_GUI_ACTIVE"] / XCC_COUNT
        quads = simds * cycles / 4
        n_el = kernel_elements(H, w, dom)
        roof["valu"] = {"frac": round((active - dual) / quads, 4),
                        "issue_quads": int(active - dual), "simd_quads": int(quads),
                        "dual_issue_share": round(dual / max(1.0, active), 4),
                        "wave_instructions": int(winst), "cycles": int(cycles),
                        "lane_instructions_per_element": round(winst * 64 / n_el, 1) if n_el >= 65536 else None,
                        "clock_ghz_implied": round(cycles / (dom_avg_ms * 1e-3) / 1e9, 3),
                        "how": "(SQ_ACTIVE_INST_VALU - SQ_ACTIVE_INST_VALU2) / (SIMDs x GRBM_GUI_ACTIVE/8 / 4), "
                               "one rocprofv3 pass: the share of SIMD issue quad-cycles with VALU work"}
        # per element of the kernel's largest non-scratch operand; a kernel
        # whose operands are all small (a reduction of values generated in
        # the kernel) has no such count
        classes = {c[len("SQ_INSTS_VALU_"):].lower(): round(dc[c] * 64 / n_el, 2)
                   for c in VALU_CLASSES if c in dc} if n_el >= 65536 else {}
        if classes:
            roof["valu"]["lane_instructions_per_element_by_class"] = classes
        if args.config in ("poly", "poly64"):
            from cudacaml_amd.examples import refbench as RB

            roof["valu"]["achieved_tflops"] = round(RB.N * RB.poly_flops() / (dom_avg_ms * 1e-3) / 1e12, 2)
    if args.config in MFMA_CONFIGS and "SQ_VALU_MFMA_BUSY_CYCLES" in dc and dc.get("GRBM_GUI_ACTIVE"):
        # Matrix cores: busy cycles per SIMD over the dispatch's cycles
        # (rocprofv3's MfmaUtil), and the math operations the matrix cores
        # counted (512 flops per MOPS unit) per clock against the peak per
        # clock, both from one pass.
        cycles = dc["GRBM_GUI_ACTIVE"] / XCC_COUNT
        mops = dc.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0) + dc.get("SQ_INSTS_VALU_MFMA_MOPS_F64", 0.0)
        cflops = mops * 512
        peak_tf = roof["peak"]
        roof["mfma"] = {"busy_frac": round(dc["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * cycles), 4),
                        "counter_flops": int(cflops), "cycles": int(cycles),
                        "counter_flops_vs_2mnk": round(cflops / roof["flops_per_launch"], 4),
                        "frac_per_clock": round(cflops / cycles / (peak_tf * 1e12 / MFMA_CLOCK_HZ), 4),
                        "clock_ghz_implied": round(cycles / (dom_avg_ms * 1e-3) / 1e9, 3),
                        "how": "busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE/8); flops = 512 x "
                               "SQ_INSTS_VALU_MFMA_MOPS_F32/F64; frac_per_clock against peak / 2.4 GHz; one pass"}
    roof["kernel"] = dom
    roof["template"] = dom_role
    roof["algorithmic_bytes"] = dom_bytes
    if dom_root_bytes != dom_bytes:
        roof["root_bytes"] = dom_root_bytes
    roof["launches"] = len(each)
    roof["launch_ms"] = round(dom_avg_ms, 4)
    if each:
        roof["launch_ms_best"] = round(min(each), 4)
        roof["launch_ms_median"] = round(statistics.median(each), 4)
    roof["traffic_detail"] = traffic_detail
    # the other kernels that move a root's bytes: counter traffic per launch
    # beside the bytes each moves, from the same counter passes
    others = []
    for k, (role, moved, _, _) in sorted(kinfo.items()):
        if k == dom or moved <= 0:
            continue
        t, _ = traffic_of(counters, k)
        if t is not None:
            others.append({"kernel": k, "template": role, "moved_bytes": moved, "traffic": t})
    if others:
        roof["other_kernels"] = others

    whole = None
    vs_baseline, vs_basis = None, None
    if args.config in BS_CONFIGS:
        ms = whole_run_ms(H, w, reps=5, mean=True)
        whole = {"ms": round(ms, 4),
                 "what": "host scalars in, host scalars out: run after one warm run, mean of 5 (as S20)"}
        if args.config in BS_PUBLISHED_MS:
            pub = BS_PUBLISHED_MS[args.config]
            whole["published_a100_ms"] = pub
            vs_baseline = round(pub / ms, 3)
            vs_basis = ("whole-run paths/s against the reference's published A100 S20 time "
                        "(%.1f ms, README.md:152-157); same graph, size and timing method" % pub)
    elif args.config in ("poly", "poly64") and not args.no_whole_run:
        from cudacaml_amd.examples import refbench as RB
        from cudacaml_amd.ir import F32, F64

        dts = "f64" if args.config == "poly64" else "f32"
        whole = refbench_whole_runs(H, F64 if dts == "f64" else F32, pinned=args.pinned)
        whole["what"] = ("the reference benchmark's RESULT fields, measured as bench/bench.ml:227-300 does: "
                         "best of 5 whole runs, host arrays in and out")
        pub = RB.PUBLISHED_A100[dts]
        whole["published_a100"] = pub
        whole["ms"] = round(whole["poly_cuda_s"] * 1e3, 3)
        vs_baseline = round(whole["poly_gflops"] / pub["poly_gflops"], 3)
        vs_basis = ("whole-run poly GFLOP/s against the reference's published A100-SXM4-40GB figure "
                    "(%.2f GFLOP/s, bench/results/nvidia-a100-sxm4-40gb.md:36-37); same graph, inputs, size "
                    "and timing method" % pub["poly_gflops"])
    elif not args.no_whole_run:
        whole = {"ms": round(whole_run_ms(H, w), 2),
                 "what": "host arrays in, host arrays out: upload + kernels + download, pageable memory"}

    cpu = None
    if not args.no_cpu:
        v, unit, sample, secs = cpu_baseline(args.config, C, H, w)
        cpu = {"value": float("%.4g" % v), "unit": unit, "cores": 1, "kind": "port",
               "sample": sample + " (%.1fs, C restatement of the OCaml interpreter, one thread)" % secs,
               "host_cpu": host_cpu()}

    line = {
        "metric": "HBM GB/s & % peak (fused map/reduce/scan); matmul TFLOP/s; MC paths/s",
        "value": round(value, 2),
        "unit": w.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": vs_baseline,
        "dtype": w.dtype,
        "data": "synthetic (Philox-4x32-10 inputs generated on the device)",
        "config": {"workload": w.describe, "parallelism": "single GPU", "moved_bytes_per_step": moved_total,
                   "plan_bytes_per_step": plan_total,
                   "plan_gbs": round(plan_total * args.steps / elapsed / 1e9, 2)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "whole_run": whole,
    }
    if vs_basis:
        line["vs_baseline_basis"] = vs_basis
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
