"""The runtime and executor on the device, as the reference's GPU unit
suites test them: test_runtime.ml (a hand-written kernel end to end),
test_info.ml, test_pool.ml (S5), test_streams.ml (S15/S16), test_pinned.ml
(S18) and the GPU half of test_executor.ml, plus S14 (f32 Greeks against
the closed form)."""

import math

import numpy as np
import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff
from cudacaml_amd import grad as G
from cudacaml_amd.examples import black_scholes as bs
from cudacaml_amd.examples import programs as P
from cudacaml_amd.examples import saxpy as sx
from cudacaml_amd.ir import F32, F64, Graph
from cudacaml_amd.runtime import Buffer, Device, Event, Jit, Launch, Pinned, Stream

pytestmark = pytest.mark.gpu

SAXPY_SRC = """
extern "C" __global__ void saxpy(float* x, float* y, float* out) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < 1000; i += gridDim.x * blockDim.x)
    out[i] = 2.0f * x[i] + y[i];
}
"""

N = 4096
SAXPY = sx.program(N, 2.0)


def inputs(k):
    return [("x", np.arange(k, N + k, dtype=np.float32)), ("y", np.ones(N, np.float32))]


def expect(k):
    return float(np.sum(2.0 * np.arange(k, N + k, dtype=np.float64) + 1.0))


def scalar(outs, name):
    return float(np.asarray(dict(outs)[name]).reshape(-1)[0])


# ---- test_runtime.ml --------------------------------------------------------


def test_init_idempotent_and_name(device):
    Device.init()
    Device.init()
    assert len(Device.name()) > 0


def test_alloc_free_byte_size(device):
    b = Buffer.alloc(4096)
    assert b.byte_size() == 4096
    b.free()


def test_upload_download_roundtrip_and_size_check(device):
    v = np.array([1, 2, 3, 4], np.int32)
    b = Buffer.alloc(16)
    b.upload(v)
    w = np.zeros(4, np.int32)
    b.download(w)
    assert w.tolist() == [1, 2, 3, 4]
    with pytest.raises(ValueError):
        b.upload(np.zeros(4, np.float64))
    b.free()
    small = Buffer.alloc(8)
    with pytest.raises(ValueError):
        small.upload(np.zeros(4, np.float32))
    small.free()


def test_jit_exposes_kernel_by_name(device):
    """The HIP counterpart of ``.entry saxpy`` in the PTX: a code object and
    a kernel that resolves by name; an unknown name raises."""
    m = Jit.compile("saxpy", SAXPY_SRC)
    assert Jit.code_size(m) > 0
    assert Jit.get_kernel(m, "saxpy")
    with pytest.raises(RuntimeError):
        Jit.get_kernel(m, "nope")
    Jit.unload(m)


def test_jit_compile_error_raises(device):
    with pytest.raises(RuntimeError, match="hiprtc"):
        Jit.compile("bad", "this is not hip")


def test_hand_written_saxpy_end_to_end(device):
    n = 1000
    x = np.arange(n, dtype=np.float32)
    y = (n - np.arange(n)).astype(np.float32)
    bx, by, bo = Buffer.alloc(4 * n), Buffer.alloc(4 * n), Buffer.alloc(4 * n)
    bx.upload(x)
    by.upload(y)
    m = Jit.compile("saxpy", SAXPY_SRC)
    Launch.run(Jit.get_kernel(m, "saxpy"), grid=4, block=256, bufs=[bx, by, bo])
    Device.synchronize()
    out = np.zeros(n, np.float32)
    bo.download(out)
    np.testing.assert_array_equal(out, 2.0 * x + y)
    for b in (bx, by, bo):
        b.free()
    Jit.unload(m)


# ---- test_info.ml -----------------------------------------------------------


def test_info_fields_and_rendering(device):
    i = Device.info()
    assert len(i.name) > 0 and i.arch.startswith("gfx950")
    assert i.multiprocessors >= 1 and i.total_memory_bytes >= 1 << 30
    lines = Device.info_to_string(i).strip().split("\n")
    assert len(lines) == 4
    assert lines[0].startswith("device: ")
    assert lines[1] == "compute: %s" % i.arch
    assert lines[2] == "multiprocessors: %d" % i.multiprocessors
    assert lines[3] == "memory_mib: %d" % (i.total_memory_bytes // 1048576)
    assert Device.name() == i.name
    assert Device.count() >= 1 and Device.current() == 0
    with Device.with_device(0):
        assert Device.current() == 0


# ---- test_pool.ml (S5) ------------------------------------------------------


def test_pool_allocated_at_compile_and_stable_over_50_runs(device):
    before = Buffer.live_count()
    c = H.compile(SAXPY)
    held = H.executor(c).buffer_count()
    assert held >= 4
    assert Buffer.live_count() == before + held
    for k in range(1, 51):
        s = scalar(H.run(c, inputs(k)), "s")
        e = expect(k)
        assert abs(s - e) <= e * 1e-4
        assert Buffer.live_count() == before + held
    c.release()
    assert Buffer.live_count() == before


def test_release_idempotent_and_run_after_release_raises(device):
    before = Buffer.live_count()
    c = H.compile(SAXPY)
    c.release()
    c.release()
    assert Buffer.live_count() == before
    with pytest.raises(RuntimeError):
        H.run(c, inputs(1))


def test_two_programs_interleave(device):
    chain = P.find("chain")
    c1, c2 = H.compile(SAXPY), H.compile(chain.graph())
    want = oracle.run(chain.graph(), chain.inputs())
    for k in range(1, 6):
        e = expect(k)
        assert abs(scalar(H.run(c1, inputs(k)), "s") - e) <= e * 1e-4
        got = H.run(c2, chain.inputs())
        assert Diff.compare_all(want, got, 1e-4) == (True, None)
    c1.release()
    c2.release()


def test_outputs_of_successive_runs_are_distinct(device):
    c = H.compile(SAXPY)
    o1 = dict(H.run(c, inputs(1)))
    o2 = dict(H.run(c, inputs(1)))
    o1["r"][0] = -999.0
    assert float(o2["r"][0]) == 3.0
    c.release()


def test_missing_input_raises_and_leaks_nothing(device):
    c = H.compile(SAXPY)
    live = Buffer.live_count()
    with pytest.raises(ValueError):
        H.run(c, [("x", np.arange(N, dtype=np.float32))])
    with pytest.raises(ValueError):
        H.run(c, [("x", np.arange(N, dtype=np.float32)), ("y", np.ones(N - 1, np.float32))])
    assert Buffer.live_count() == live
    c.release()


# ---- test_executor.ml, GPU half ---------------------------------------------


def test_executor_runs_twice_with_different_inputs(device):
    e = P.sum_(100)
    c = H.compile(e.graph())
    assert abs(scalar(H.run(c, [("x", np.full(100, 1.0, np.float32))]), "s") - 100.0) <= 1e-3
    assert abs(scalar(H.run(c, [("x", np.full(100, 2.0, np.float32))]), "s") - 200.0) <= 1e-3
    c.release()


# ---- test_streams.ml (S15/S16) ----------------------------------------------


def test_streams_and_events(device):
    s = Stream.create()
    e0 = Event.record(Stream.default)
    e1 = Event.record(s)
    e1.synchronize()
    s.synchronize()
    e0.synchronize()
    assert s.is_idle()
    assert Event.elapsed_ms(e0, e1) == Event.elapsed_ms(e0, e1)  # both complete: a number, no error
    e2 = Event.record(Stream.default)
    e2.synchronize()
    assert Event.elapsed_ms(e0, e2) >= 0.0


def test_async_jobs_on_three_streams_equal_sync(device):
    c = H.compile_with(3, SAXPY)
    jobs = [(k, H.run_async(c, inputs(k))) for k in range(8)]
    for k, j in jobs:
        got = dict(H.wait(j))
        want = dict(H.run(c, inputs(k)))
        np.testing.assert_array_equal(got["r"], want["r"])
        assert float(got["s"]) == float(want["s"])
    j = H.run_async(c, inputs(99))
    a, b = dict(H.wait(j)), dict(H.wait(j))
    assert float(a["s"]) == float(b["s"])
    c.release()


def test_resident_roundtrip(device):
    v = (np.arange(1000) * 0.25).astype(np.float32)
    r = H.upload(v)
    assert tuple(r.shape) == (1000,)
    np.testing.assert_array_equal(H.download(r), v)
    H.free_resident(r)


def test_run_resident_equals_host_run(device):
    c = H.compile(SAXPY)
    ins = inputs(3)
    rx, ry = H.upload(ins[0][1]), H.upload(ins[1][1])
    outs = dict(H.run_resident(c, [("x", rx), ("y", ry)]))
    want = dict(H.run(c, ins))
    rr, rs = outs["r"], outs["s"]
    assert tuple(rr.shape) == (N,) and tuple(rs.shape) == () and rr.dtype is F32
    np.testing.assert_array_equal(H.download(rr), want["r"])
    assert float(H.download(rs)) == float(want["s"])
    for r in (rx, ry, rr, rs):
        H.free_resident(r)
    c.release()


def test_resident_chaining_without_host_round_trip(device):
    before = Buffer.live_count()
    chain = P.find("chain")
    gc, gs = chain.graph(), P.sum_(4096).graph()
    cc, cs = H.compile(gc), H.compile(gs)
    rx = H.upload(dict(chain.inputs())["x"])
    r = dict(H.run_resident(cc, [("x", rx)]))["r"]
    s = dict(H.run_resident(cs, [("x", r)]))["s"]
    got = float(H.download(s))
    want = scalar(oracle.run(gs, [("x", dict(oracle.run(gc, chain.inputs()))["r"])]), "s")
    assert abs(got - want) <= 1e-4 * (1.0 + abs(want))
    for x in (rx, r, s):
        H.free_resident(x)
    cc.release()
    cs.release()
    assert Buffer.live_count() == before


# ---- test_pinned.ml (S18) ---------------------------------------------------


def test_pinned_alloc_is_pinned(device):
    v = Pinned.alloc(F32, (1000,))
    assert v.size == 1000
    v[:] = np.arange(1000)
    assert float(v[999]) == 999.0
    assert Pinned.is_pinned(v)
    assert not Pinned.is_pinned(np.zeros(4, np.float32))


def test_pinned_in_and_out_through_a_device_buffer(device):
    n = 1 << 24
    src, dst = Pinned.alloc(F32, (n,)), Pinned.alloc(F32, (n,))
    src[:] = (np.arange(n) & 1023).astype(np.float32)
    b = Buffer.alloc(src.nbytes)
    b.upload(src)
    b.download(dst)
    b.free()
    np.testing.assert_array_equal(src, dst)


def test_pinned_inputs_through_run_and_run_async(device):
    x, y = Pinned.alloc(F32, (N,)), Pinned.alloc(F32, (N,))
    x[:] = np.arange(N)
    y[:] = 1.0
    c = H.compile_with(2, SAXPY)
    s = scalar(H.run(c, [("x", x), ("y", y)]), "s")
    e = expect(0)
    assert abs(s - e) <= e * 1e-4
    jobs = [H.run_async(c, [("x", x), ("y", y)]) for _ in range(4)]
    for j in jobs:
        assert scalar(H.wait(j), "s") == s
    c.release()


def test_pinned_memory_is_freed_when_dropped(device):
    for _ in range(50):
        Pinned.alloc(F32, (256 * 1024,))
    import gc

    gc.collect()
    Pinned.alloc(F32, (256 * 1024,))


# ---- the pinned staging block of a synchronous run -----------------------------


def test_small_values_through_the_staging_block(device):
    """Params and outputs of at most 4 KiB and the error word travel through
    one pinned block per synchronous run: an output that is a param, one
    value under two names, small and large outputs side by side, a gather's
    error raised and cleared; run, run_async and the oracle agree."""
    from cudacaml_amd import dsl as D
    from cudacaml_amd.ir import I32

    x = D.param("x", F32, (5,))
    y = D.param("y", F32, (100000,))
    i = D.param("i", I32, (3,))
    s = D.reduce(D.add, D.const(F32, 0.0), y)
    g = Graph.create("stage", [("x", x), ("s", s), ("s2", s), ("r", D.map(lambda v: D.mul(v, D.const(F32, 2.0)), x)),
                               ("ny", D.map(D.neg, y)), ("gx", D.gather(i, x))])
    c = H.compile_with(2, g)
    try:
        for k in range(3):
            ins = [("x", np.arange(k, k + 5, dtype=np.float32)),
                   ("y", np.linspace(0.5, 1 + k, 100000, dtype=np.float32)),
                   ("i", np.array([4, 0, k], np.int32))]
            want = oracle.run(g, ins)
            got = H.run(c, ins)
            assert [n for n, _ in got] == ["x", "s", "s2", "r", "ny", "gx"]
            same, msg = Diff.compare_all(want, got, 1e-4)
            assert same, msg
            assert float(dict(got)["s"]) == float(dict(got)["s2"])
            asy = H.wait(H.run_async(c, ins))
            for (n, a), (_, b) in zip(got, asy):
                np.testing.assert_array_equal(a, b, err_msg=n)
        bad = [("x", np.zeros(5, np.float32)), ("y", np.zeros(100000, np.float32)), ("i", np.array([0, 5, 1], np.int32))]
        with pytest.raises(ValueError, match="gather index out of bounds"):
            H.run(c, bad)
        ok = dict(H.run(c, ins))
        assert ok["gx"].tolist() == [float(k + 4), float(k), float(k + 2)]
    finally:
        c.release()


@pytest.mark.parametrize("streams", [1, 2])
def test_async_errors_stay_with_their_job(device, streams):
    """Jobs queued on one lane (and on a ring of two) each report only
    their own device-side index error: a clean job queued before a bad one
    waits cleanly even when the bad one has finished first, the bad one
    raises, and later runs start from a clear error word."""
    from cudacaml_amd import dsl as D
    from cudacaml_amd.ir import I32

    n = 1 << 16
    x = D.param("x", F32, (n,))
    i = D.param("i", I32, (n,))
    g = Graph.create("gx", [("g", D.gather(i, x))])
    xv = np.arange(n, dtype=np.float32)
    good = [("x", xv), ("i", (np.arange(n)[::-1] % n).astype(np.int32))]
    badi = good[1][1].copy()
    badi[n // 2] = n + 7
    bad = [("x", xv), ("i", badi)]
    c = H.compile_with(streams, g)
    try:
        jobs = [H.run_async(c, good), H.run_async(c, bad), H.run_async(c, good), H.run_async(c, bad),
                H.run_async(c, good)]
        # the last job done first: every earlier job on its lane is done too
        H.wait(jobs[-1])
        for k in (0, 2):
            np.testing.assert_array_equal(dict(H.wait(jobs[k]))["g"], xv[good[1][1]])
        for k in (1, 3):
            with pytest.raises(ValueError, match="gather index out of bounds"):
                H.wait(jobs[k])
            with pytest.raises(ValueError, match="gather index out of bounds"):
                H.wait(jobs[k])  # a second wait reports the same outcome
        np.testing.assert_array_equal(dict(H.run(c, good))["g"], xv[good[1][1]])
        with pytest.raises(ValueError, match="gather index out of bounds"):
            H.run(c, bad)
        np.testing.assert_array_equal(dict(H.wait(H.run_async(c, good)))["g"], xv[good[1][1]])
    finally:
        c.release()


# ---- recorded launch sequences (HIP graphs) ------------------------------------


def _eager_and_graphed(monkeypatch, g, streams=1):
    monkeypatch.setenv("CCHIP_TUNE", "graphs=0")
    eager = H.compile_with(streams, g)
    monkeypatch.setenv("CCHIP_TUNE", "graphs=1")
    graphed = H.compile_with(streams, g)
    monkeypatch.delenv("CCHIP_TUNE")
    return eager, graphed


def _same(a, b):
    assert [n for n, _ in a] == [n for n, _ in b]
    for (n, x), (_, y) in zip(a, b):
        np.testing.assert_array_equal(np.asarray(x), np.asarray(y), err_msg=n)


def test_graph_replays_equal_eager_launches(device, monkeypatch):
    """A program of many kernels (the Greeks adjoint, 25 launches) replayed
    from its recorded graph gives, on every replay, exactly what eager
    launches give: host runs with eager work and synchronisation between
    the replays, async runs on a ring of lanes, and resident runs whose
    output buffers change (each pointer set records its own graph, and more
    sets than the cache holds evict the oldest)."""
    from cudacaml_amd.runtime import Buffer, Device

    g = bs.call_greeks(1 << 16, F32)
    eager, graphed = _eager_and_graphed(monkeypatch, g, streams=2)
    try:
        for seed in (1, 2, 3, 1):
            ins = bs.inputs(F32, seed=seed)
            want = H.run(eager, ins)
            _same(want, H.run(graphed, ins))
            Device.synchronize()
            _same(want, H.wait(H.run_async(graphed, ins)))
        ins = bs.inputs(F32, seed=5)
        want = H.run(eager, ins)
        res_in = [(n, H.upload(v)) for n, v in ins]
        sets = []
        for k in range(11):
            outs = [(o.name, H.Resident(Buffer.alloc(o.nbytes), o.dtype, o.shape)) for o in graphed.outputs]
            sets.append(outs)
            H.run_resident_into(graphed, res_in, outs, sync=(k % 3 == 0))
        Device.synchronize()
        for outs in sets + sets[:2]:
            H.run_resident_into(graphed, res_in, outs, sync=True)
            _same(want, [(n, H.download(r)) for n, r in outs])
        for outs in sets:
            for _, r in outs:
                H.free_resident(r)
        for _, r in res_in:
            H.free_resident(r)
    finally:
        eager.release()
        graphed.release()


def test_graph_replays_of_a_look_back_scan(device, monkeypatch):
    """The look-back scan's status words are cleared by its own fill kernel
    in every replay: repeated graphed runs stay bit-exact (i32)."""
    from cudacaml_amd import dsl as D
    from cudacaml_amd.ir import I32

    n = 3 * (1 << 20) + 7
    g = Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 5), D.param("x", I32, (1, n))))])
    eager, graphed = _eager_and_graphed(monkeypatch, g)
    try:
        for seed in (11, 12, 11):
            ins = [("x", _small_ints(seed, n).reshape(1, n))]
            want = H.run(eager, ins)
            for _ in range(3):
                _same(want, H.run(graphed, ins))
    finally:
        eager.release()
        graphed.release()


def _small_ints(seed, n):
    from cudacaml_amd.examples import configs as C

    return C.small_ints(seed, (n,))


# ---- S14 --------------------------------------------------------------------


def test_s14_bs_greeks_f32_vs_closed_form(device):
    cf = bs.analytic()
    c = H.compile(bs.call_greeks(1 << 20, F32))
    o = H.run(c, bs.inputs(F32, seed=3))
    c.release()

    def g(w):
        return bs.scalar_out(o, G.grad_name("price", w))

    assert abs(bs.scalar_out(o, "price") - cf["price"]) <= 0.1
    assert abs(g("s0") - cf["delta"]) <= 0.01
    assert abs(g("vol") - cf["vega"]) <= 0.6
    assert math.isfinite(g("rate"))


# ---- S20 --------------------------------------------------------------------


def test_s20_timing_table(device, capsys):
    """The reference's S20 row (test_system.ml:225-245): the one-step price
    and its Greeks adjoint at 2^22 paths, f32 and f64, each run once warm
    and then timed as the mean of 5 host-to-host runs. Informational, as
    there; the prices are checked against the closed form."""
    import time

    n = 1 << 22
    cf = bs.analytic()
    rows = []
    for dt in (F32, F64):
        ins = bs.inputs(dt, seed=1)
        times = []
        for g in (bs.call_mc(n, dt), bs.call_greeks(n, dt)):
            c = H.compile(g)
            o = H.run(c, ins)
            t0 = time.perf_counter()
            for _ in range(5):
                o = H.run(c, ins)
            times.append((time.perf_counter() - t0) / 5.0)
            c.release()
            assert abs(bs.scalar_out(o, "price") - cf["price"]) <= 0.1
        rows.append((dt.name, times[0], times[1]))
    with capsys.disabled():
        for name, tp, tg in rows:
            print("\n    %s  price %.3f ms   greeks %.3f ms   ratio %.2fx" % (name, tp * 1e3, tg * 1e3, tg / tp))
