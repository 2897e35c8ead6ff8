"""The allocation-free entry point, cchip_program_run_resident_noalloc: the
template scratch comes from the library's static device array, the work
runs on a stream the caller chooses, and no device memory is allocated.

Every call is checked against the existing run_resident_into on the same
program and the same inputs, bit for bit (the outputs here are integer
scans and scatters, a max scan and a fixed-order split reduction, all
exactly reproducible), over calls in a row whose programs lay the static
scratch out differently: a program that uses 28 of its 32 MiB (two
look-back scans, a split reduction, a sliced scatter), then a smaller one
(the direct scatter), then the first again with other inputs."""

import math

import numpy as np
import pytest

from cudacaml_amd import backend_hip as H
from cudacaml_amd import dsl as D
from cudacaml_amd.ir import F32, I32, Graph
from cudacaml_amd.runtime import Buffer, Stream

pytestmark = pytest.mark.gpu


def program(n, bins):
    v = D.param("v", I32, (n,))
    x = D.param("x", F32, (n,))
    idx = D.param("idx", I32, (n,))
    w = D.param("w", I32, (n,))
    p = D.scan(D.add, D.const(I32, 0), v)
    return Graph.create("noalloc", [
        ("p", p),
        ("m", D.scan(D.max, D.const(F32, -math.inf), x)),
        ("t", D.reduce(D.add, D.const(F32, 0.0), x)),
        ("h", D.scatter_add(idx, w, (bins,))),
        ("v", v),    # an output that is a param: copied
        ("p2", p),   # one buffer under two names: copied
    ])


def inputs(n, bins, seed):
    r = np.random.default_rng(seed)
    return [("v", r.integers(-9, 17, n, dtype=np.int32)),
            ("x", r.standard_normal(n).astype(np.float32)),
            ("idx", r.integers(0, bins, n, dtype=np.int32)),
            ("w", r.integers(-3, 8, n, dtype=np.int32))]


def scratch_bytes(g):
    size = {"f32": 4, "i32": 4, "f64": 8, "i64": 8}
    tot = 0
    for line in H.plan(g).splitlines():
        f = line.split()
        if f[0] == "buffer" and f[5] == "scratch":
            tot += (max(int(f[4]) * size[f[3]], 1) + 255) // 256 * 256
    return tot


def outputs_of(c):
    return [(o.name, H.Resident(Buffer.alloc(o.nbytes), o.dtype, o.shape)) for o in c.outputs]


def free_all(rs):
    for _, r in rs:
        H.free_resident(r)


def check_call(c, ins, stream):
    """One allocation-free call against run_resident_into on the same
    inputs; also against numpy for the integer outputs."""
    res = [(n, H.upload(v)) for n, v in ins]
    want_o, got_o = outputs_of(c), outputs_of(c)
    try:
        H.run_resident_into(c, res, want_o, sync=True)
        live = Buffer.live_count()
        H.run_resident_noalloc(c, res, got_o, stream.ptr)
        stream.synchronize()
        assert Buffer.live_count() == live
        want = {n: H.download(r) for n, r in want_o}
        got = {n: H.download(r) for n, r in got_o}
        for name in want:
            np.testing.assert_array_equal(got[name], want[name], err_msg=name)
        v = dict(ins)
        np.testing.assert_array_equal(got["p"], np.cumsum(v["v"], dtype=np.int64).astype(np.int32))
        np.testing.assert_array_equal(got["p2"], got["p"])
        np.testing.assert_array_equal(got["v"], v["v"])
        np.testing.assert_array_equal(got["m"], np.maximum.accumulate(v["x"]))
        bins = c.outputs[3].shape[0]
        np.testing.assert_array_equal(got["h"], np.bincount(v["idx"], weights=v["w"], minlength=bins).astype(np.int32))
    finally:
        free_all(res)
        free_all(want_o)
        free_all(got_o)


@pytest.mark.parametrize("on", ["created", "default"])
def test_noalloc_calls_in_a_row_match_run_resident_into(device, on):
    big, small = ((1 << 22), 1 << 16), ((1 << 20) + 3, 1 << 12)
    ga, gb = program(*big), program(*small)
    assert 24 << 20 < scratch_bytes(ga) <= 32 << 20
    assert 0 < scratch_bytes(gb) < scratch_bytes(ga)
    stream = Stream.create() if on == "created" else Stream.default
    ca, cb = H.compile(ga), H.compile(gb)
    try:
        check_call(ca, inputs(*big, seed=1), stream)
        check_call(cb, inputs(*small, seed=2), stream)
        check_call(ca, inputs(*big, seed=3), stream)
    finally:
        ca.release()
        cb.release()


def test_noalloc_folded_sum_calls_in_a_row(device):
    """A map whose output the next root sums: the sum is folded inside the
    map kernel, so its wave partials and flags are scratch live across two
    roots. Two calls in a row, the second smaller (8192 partials folded by
    one workgroup of 1024 threads, then 512 by one of 256), each bit for
    bit against run_resident_into and numpy (integers: exact in any
    order)."""
    def prog(n):
        x, y = D.param("x", I32, (n,)), D.param("y", I32, (n,))
        r = D.map2(lambda a, b: D.add(D.mul(a, D.const(I32, 3)), b), x, y)
        return Graph.create("nafold", [("r", r), ("s", D.reduce(D.add, D.const(I32, 7), r))])

    stream = Stream.create()
    for n, seed in (((1 << 21) + 3, 5), ((1 << 17) + 1, 6)):
        g = prog(n)
        roles = [l.split()[2] for l in H.plan(g).splitlines() if l.startswith("kernel")]
        assert roles == ["map", "reduce_split_fold"], roles
        r = np.random.default_rng(seed)
        ins = [("x", r.integers(-1000, 1000, n, dtype=np.int32)), ("y", r.integers(-1000, 1000, n, dtype=np.int32))]
        c = H.compile(g)
        res = [(nm, H.upload(v)) for nm, v in ins]
        want_o, got_o = outputs_of(c), outputs_of(c)
        try:
            H.run_resident_into(c, res, want_o, sync=True)
            live = Buffer.live_count()
            H.run_resident_noalloc(c, res, got_o, stream.ptr)
            stream.synchronize()
            assert Buffer.live_count() == live
            want = {nm: H.download(o) for nm, o in want_o}
            got = {nm: H.download(o) for nm, o in got_o}
            for nm in want:
                np.testing.assert_array_equal(got[nm], want[nm], err_msg=nm)
            exp_r = ins[0][1].astype(np.int64) * 3 + ins[1][1]
            np.testing.assert_array_equal(got["r"], exp_r.astype(np.int32))
            exp_s = np.array(7 + int(exp_r.sum()), dtype=np.int64).astype(np.int32)  # wrapping int32 sum
            assert int(got["s"]) == int(exp_s)
        finally:
            free_all(res)
            free_all(want_o)
            free_all(got_o)
            c.release()


def test_noalloc_rejects_programs_beyond_the_static_scratch(device):
    n, bins = 1 << 23, 1 << 20
    g = program(n, bins)
    assert scratch_bytes(g) > 32 << 20
    c = H.compile(g)
    res = [(nm, H.upload(v)) for nm, v in inputs(n, bins, seed=4)]
    outs = outputs_of(c)
    try:
        live = Buffer.live_count()
        with pytest.raises(ValueError, match="static scratch"):
            H.run_resident_noalloc(c, res, outs)
        assert Buffer.live_count() == live
        with pytest.raises(ValueError, match="missing input"):
            H.run_resident_noalloc(c, res[:2], outs)
    finally:
        free_all(res)
        free_all(outs)
        c.release()
    with pytest.raises(RuntimeError, match="released"):
        H.run_resident_noalloc(c, res, outs)


def test_noalloc_index_errors_stay_with_the_call(device):
    """An out-of-range scatter index in an allocation-free call is reported
    through that call's own error word (the caller's err buffer), and
    never by a later run: a clean synchronous run_resident_into and a clean
    run_async job on the same program succeed afterwards, and a clean
    allocation-free call returns a zero word (the scratch's word was
    cleared at the start of the call). The kernels bounds-check the index
    and skip it, as in test_scatter_out_of_range_raises."""
    n, bins = (1 << 16) + 5, 1 << 12
    c = H.compile(program(n, bins))
    bad = inputs(n, bins, seed=7)
    bad[2][1][[3, n - 2]] = [bins, -1]
    good = inputs(n, bins, seed=8)
    res_bad = [(nm, H.upload(v)) for nm, v in bad]
    res_good = [(nm, H.upload(v)) for nm, v in good]
    outs, want_o = outputs_of(c), outputs_of(c)
    err = Buffer.alloc(4)
    stream = Stream.create()
    try:
        H.run_resident_noalloc(c, res_bad, outs, stream.ptr, err=err)
        stream.synchronize()
        code = _word(err)
        assert code & 2, code
        with pytest.raises(ValueError, match="scatter_add index out of bounds"):
            H.raise_error_word(code)
        # later runs of the same program do not see the call's flags
        H.run_resident_into(c, res_good, want_o, sync=True)
        H.wait(H.run_async(c, good))
        H.run_resident_noalloc(c, res_good, outs, stream.ptr, err=err)
        stream.synchronize()
        assert _word(err) == 0
        H.raise_error_word(0)
        for (nm, w), (_, g) in zip(want_o, outs):
            np.testing.assert_array_equal(H.download(g), H.download(w), err_msg=nm)
        # and without an err buffer the flags are dropped, not passed on
        H.run_resident_noalloc(c, res_bad, outs, stream.ptr)
        stream.synchronize()
        H.run_resident_into(c, res_good, want_o, sync=True)
        H.run(c, good)
    finally:
        err.free()
        free_all(res_bad)
        free_all(res_good)
        free_all(outs)
        free_all(want_o)
        c.release()


def _word(buf):
    out = np.zeros(1, np.int32)
    buf.download(out)
    return int(out[0])
