"""Parity at the sizes bench.py times: every BASELINE config at its full
size on the device, checked through properties that hold at any size
(textbook routines on the host, closed forms, exact permutations), and
config 5's Greeks graph against the oracle at 64 steps.

Inputs are the benchmark's own: generated on the device by the build's
Philox (``configs.gen_*``), downloaded, and pinned against the host
restatement of the same formula at three sample ranges, so a test checks
exactly what the benchmark runs.

Reference: BASELINE.json configs 2-5; test/system/test_system.ml:72-75 (S3,
a multi-kernel size), examples/black_scholes.ml:116-145 and
lib/ad/grad.ml:258-281 (the Greeks graph and its scan and gather adjoints).
"""

import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff
from cudacaml_amd import dsl as D
from cudacaml_amd import grad as G
from cudacaml_amd import rng
from cudacaml_amd.examples import black_scholes as bs
from cudacaml_amd.examples import configs as C
from cudacaml_amd.ir import F32, F64, I32, Graph

pytestmark = pytest.mark.gpu

SAMPLE = 4096


def run_dev(g, inputs):
    c = H.compile(g)
    try:
        return dict(H.run(c, inputs))
    finally:
        c.release()


def gen(gen_graph, seed):
    """A synthetic input as bench.py makes it: on the device."""
    return run_dev(gen_graph, [("seed", np.array(seed, np.int32))])["v"]


def pin(v, seed, expect, exact=True, rtol=0.0):
    """The device-generated input equals the host formula over the
    Philox words at the start, a third of the way in, and the end."""
    flat = v.reshape(-1)
    n = flat.size
    for start in (0, n // 3 + 17, n - SAMPLE):
        want = expect(C.philox_w0(seed, SAMPLE, start))
        got = flat[start:start + SAMPLE]
        if exact:
            np.testing.assert_array_equal(got, want, err_msg="generator at %d" % start)
        else:
            np.testing.assert_allclose(got, want, rtol=rtol, atol=rtol, err_msg="generator at %d" % start)


def uniform_of(w):
    return ((w >> 8).astype(np.int64) - (1 << 23)).astype(np.float32) * np.float32(2.0 ** -23)


def normal_of(dtype):
    def f(w):
        from scipy.special import erfinv

        u = (w.astype(np.float64) + 0.5) * 2.0 ** -32
        return (math.sqrt(2.0) * erfinv(2.0 * u - 1.0)).astype(dtype.np)
    return f


def roles(g):
    return [l.split()[2] for l in H.plan(g).splitlines() if l.startswith("kernel")]


def band(got, exact, tol):
    """max of |got - exact| / (1 + |exact|), the policy's relative band."""
    g = np.asarray(got, dtype=np.float64)
    e = np.asarray(exact, dtype=np.float64)
    return float(np.max(np.abs(g - e) / (1.0 + np.abs(e)))) if g.size else 0.0


# ---- config 1: saxpy and the 5-map chain -----------------------------------------


def test_config1_saxpy_2_24_as_benchmarked(device):
    """The saxpy graph bench.py times, on its own inputs (x seed 1, y seed
    2, n = 2^24): r bit for bit against the oracle (one rounding per op,
    R1); s within the f32 reduction band of the exact sum of r (math.fsum
    over the f32 values of r). The oracle's own s, a sequential f32 fold
    over 2^24 terms, is checked against the same exact sum; the three
    distances are printed (oracle vs exact, device vs exact, device vs
    oracle), and the device must be no further from the exact sum than the
    band."""
    n = C.N1
    x = gen(C.gen_uniform_pm1((n,)), 1)
    y = gen(C.gen_uniform_pm1((n,)), 2)
    pin(x, 1, uniform_of)
    pin(y, 2, uniform_of)
    g = C.saxpy()
    assert roles(g) == ["map", "reduce_split_fold", "reduce_split_fold"]
    exp = dict(oracle.run(g, [("x", x), ("y", y)]))
    got = run_dev(g, [("x", x), ("y", y)])
    np.testing.assert_array_equal(got["r"], exp["r"])
    exact = math.fsum(exp["r"].astype(np.float64).tolist())
    d_oe = band(exp["s"], exact, 1e-4)
    d_de = band(got["s"], exact, 1e-4)
    d_do = band(got["s"], exp["s"], 1e-4)
    print("config1 s at 2^24: exact %.9g oracle %.9g device %.9g | band distance oracle-exact %.3g, "
          "device-exact %.3g, device-oracle %.3g" % (exact, float(exp["s"]), float(got["s"]), d_oe, d_de, d_do))
    assert d_de <= 1e-4


def test_config1_chain_2_24_bit_exact(device):
    """The 5-map chain ((-((x+1)^2))-1)*0.5 bench.py times, fused into one
    kernel, over its own 2^24 inputs (seed 1): bit for bit against the
    oracle, which rounds once per op."""
    n = C.N1
    x = gen(C.gen_uniform_pm1((n,)), 1)
    pin(x, 1, uniform_of)
    g = C.chain()
    assert roles(g) == ["map"]
    exp = dict(oracle.run(g, [("x", x)]))
    got = run_dev(g, [("x", x)])
    for name, e in exp.items():
        np.testing.assert_array_equal(got[name], e, err_msg=name)
    # the closed form in float64, as a check on the oracle's own formula
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(got[next(iter(exp))], (-((x64 + 1) ** 2) - 1) * 0.5, rtol=3e-7, atol=3e-7)


# ---- config 2: the headline workload ------------------------------------------


def test_config2_global_scan_2_28_bit_exact(device):
    """The 2^28 i32 inclusive scan the benchmark times (10083 look-back
    tiles, far more than are resident at once), bit for bit against the
    textbook sequential prefix sum."""
    n = C.SCAN2
    v = gen(C.gen_small_ints((n,)), 4)
    pin(v, 4, lambda w: (w >> 28).astype(np.int32))
    g = C.global_scan()
    assert roles(g) == ["scan_init", "scan_lookback"]
    got = run_dev(g, [("v", v)])["p"]
    want = np.cumsum(v, dtype=np.int64)
    assert want[-1] < 2 ** 31
    np.testing.assert_array_equal(got, want.astype(np.int32))


def test_config2_rows_8192_bit_exact(device, monkeypatch):
    """reduce_rows add and max and scan_rows add over the benchmark's
    f32[8192; 8192], with the float add and scan folded in order
    (rr_tree=1, rs_tree=0), bit for bit against the oracle's sequential
    folds."""
    monkeypatch.setenv("CCHIP_TUNE", "rr_tree=1,rs_tree=0")
    x = gen(C.gen_uniform_pm1((C.ROWS2, C.ROWS2)), 3)
    pin(x, 3, uniform_of)
    g = C.rows()
    exp = oracle.run(g, [("x", x)])
    got = run_dev(g, [("x", x)])
    for name, e in exp:
        np.testing.assert_array_equal(got[name], e, err_msg=name)


def test_config2_rows_8192_as_benchmarked(device):
    """The benchmark's graph as it runs by default: the add and the scan
    fold each row as a tree, within the band of the float64 row sums and
    prefix sums and no further from them than the oracle's in-order folds
    (whose own drift grows with the row count); the max bit for bit."""
    x = gen(C.gen_uniform_pm1((C.ROWS2, C.ROWS2)), 3)
    pin(x, 3, uniform_of)
    g = C.rows()
    assert roles(g) == ["scan_tile_fold"]
    exp = dict(oracle.run(g, [("x", x)]))
    got = run_dev(g, [("x", x)])
    e64 = x.astype(np.float64).sum(axis=1)
    assert band(got["sum"], e64, 1e-4) <= 1e-4
    assert band(got["sum"], e64, 1e-4) <= band(exp["sum"], e64, 1e-4)
    np.testing.assert_array_equal(got["max"], exp["max"])
    del e64
    c64 = np.cumsum(x.astype(np.float64), axis=1)
    assert band(got["scan"], c64, 1e-4) <= 1e-4
    assert band(got["scan"], c64, 1e-4) <= band(exp["scan"], c64, 1e-4)


# ---- config 3: scatter_add and the gather back ----------------------------------


def test_config3_scatter_gather_2_26_into_2_20(device):
    """2^26 uniform indices into 2^20 bins: each bin against the float64
    bincount within the accumulation band; the gather back exactly h[idx]."""
    idx = gen(C.gen_bin_indices(C.N3, 20), 6)
    src = gen(C.gen_uniform_pm1((C.N3,)), 5)
    pin(idx, 6, lambda w: (w >> 12).astype(np.int32))
    pin(src, 5, uniform_of)
    o = run_dev(C.scatter_gather(), [("idx", idx), ("src", src)])
    exact = np.bincount(idx, weights=src.astype(np.float64), minlength=C.BINS3)
    assert o["h"].shape == (C.BINS3,)
    assert band(o["h"], exact, 1e-4) <= 1e-4
    np.testing.assert_array_equal(o["back"], o["h"][idx])


def test_config3_permutation_2_26_bins(device):
    """The collision-free case: a permutation of 2^26 indices into 2^26
    bins (the two-level partition). Every bin receives exactly one value,
    so h is the source permuted and the gather back is the source, both
    bit for bit."""
    n = C.N3
    perm = np.random.default_rng(7).permutation(n).astype(np.int32)
    src = gen(C.gen_uniform_pm1((n,)), 5)
    g = C.scatter_gather(n, n)
    assert "scatter_coarse" in roles(g)
    o = run_dev(g, [("idx", perm), ("src", src)])
    np.testing.assert_array_equal(o["h"][perm], src)
    np.testing.assert_array_equal(o["back"], src)


# ---- config 4: matmul and its adjoint ------------------------------------------


def test_config4_matmul_f64_2048_vs_exact(device):
    """f64 2048^3 against the float64 product (whose own error is far below
    the 1e-12 band), and 64 entries against the exact rational sum."""
    n = C.MM_F64
    a = gen(C.gen_normals((n, n), F64), 8)
    b = gen(C.gen_normals((n, n), F64), 9)
    pin(a, 8, normal_of(F64), exact=False, rtol=1e-12)
    g = C.matmul(n, F64)
    assert roles(g) == ["matmul_mfma_f64_a0b0"]
    got = run_dev(g, [("a", a), ("b", b)])["c"]
    assert band(got, a @ b, 1e-12) <= 1e-12
    r = np.random.default_rng(1)
    for i, j in zip(r.integers(0, n, 64), r.integers(0, n, 64)):
        exact = float(sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(a[i], b[:, j])))
        assert abs(got[i, j] - exact) <= 1e-12 * (1 + abs(exact)), (i, j)


def test_config4_matmul_f32_4096_normals_vs_exact(device):
    """The forward f32 4096^3 product bench.py times, on its own N(0,1)
    draws (seeds 8 and 9): every entry within the f32 band of the float64
    product of the same f32 inputs (whose own error is far below it); the
    worst entry and the normwise error are printed."""
    n = C.MM_F32
    a = gen(C.gen_normals((n, n), F32), 8)
    b = gen(C.gen_normals((n, n), F32), 9)
    pin(a, 8, normal_of(F32), exact=False, rtol=2e-6)
    pin(b, 9, normal_of(F32), exact=False, rtol=2e-6)
    g = C.matmul(n, F32)
    assert roles(g) == ["matmul_mfma_f32_a0b0"]
    got = run_dev(g, [("a", a), ("b", b)])["c"].astype(np.float64)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    err = np.abs(got - exact) / (1.0 + np.abs(exact))
    print("config4 f32 4096^3 on N(0,1): max band distance %.3g at |e| = %.3g, normwise %.3g"
          % (err.max(), abs(exact.flat[err.argmax()]), np.linalg.norm(got - exact) / np.linalg.norm(exact)))
    assert err.max() <= 1e-4, err.max()


@pytest.mark.parametrize("dtype,n,tol", [(F32, C.MM_F32, 1e-4), (F64, C.MM_F64, 1e-12)], ids=["f32", "f64"])
def test_config4_matmul_grad_full_size_closed_form(device, dtype, n, tol):
    """Grad of s = sum(A@B) at the benchmark's sizes: three matmuls, two
    over transposed operands. Closed forms: ds/dA[i,p] = sum_j B[p,j],
    ds/dB[p,j] = sum_i A[i,p], s = sum_p colsum(A)_p rowsum(B)_p."""
    a = gen(C.gen_normals((n, n), dtype), 8)
    b = gen(C.gen_normals((n, n), dtype), 9)
    g = C.matmul_grad(n, dtype)
    assert {"matmul_mfma_%s_a0b1" % dtype.name, "matmul_mfma_%s_a1b0" % dtype.name} <= set(roles(g))
    o = run_dev(g, [("a", a), ("b", b)])
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    rs_b, cs_a = b64.sum(axis=1), a64.sum(axis=0)
    assert band(o["ds/da"], np.broadcast_to(rs_b, (n, n)), tol) <= tol
    assert band(o["ds/db"], np.broadcast_to(cs_a[:, None], (n, n)), tol) <= tol
    s = float(np.asarray(o["s"]).reshape(-1)[0])
    s_exact = math.fsum(cs_a * rs_b)
    assert abs(s - s_exact) <= tol * (1 + abs(s_exact)), (s, s_exact)


# ---- config 5: Black-Scholes Monte Carlo with pathwise Greeks ---------------------


@pytest.mark.parametrize("dtype", [F32, F64], ids=["f32", "f64"])
def test_config5_greeks_64_steps_vs_oracle(device, dtype):
    """Grad.grad of the 64-step path pricer (price, delta, vega) against
    the oracle under the per-output policy, at 8192 paths: the scan
    adjoint (total - prefix + abar), the gather adjoint's scatter, and
    the row reductions and scans over the adjoints."""
    g = C.mc_greeks(8192, C.STEPS5, dtype)
    ins = bs.inputs(dtype, seed=7)
    exp = oracle.run(g, ins)
    got = run_dev(g, ins)
    bad = [v for v in Diff.policy_check(g, exp, list(got.items())) if not v.ok]
    assert not bad, bad
    ok, msg = Diff.compare_all(exp, list(got.items()), 1e-4 if dtype is F32 else 1e-12)
    assert ok, msg


def pathwise(zsum, steps):
    """The hand-derived pathwise estimator with the exact GBM, from each
    path's sum of normal draws: price = e^-rT mean(max(S_T - K, 0)),
    delta = e^-rT mean(1{S_T>K} S_T/S0),
    vega = e^-rT mean(1{S_T>K} S_T (sqrt(dt) sum Z - vol T))."""
    m = bs.market
    dt = m.maturity / steps
    st = m.s0 * np.exp((m.rate - 0.5 * m.vol ** 2) * m.maturity + m.vol * math.sqrt(dt) * zsum)
    itm = st > m.strike
    disc = math.exp(-m.rate * m.maturity)
    return {
        "price": disc * np.mean(np.maximum(st - m.strike, 0.0)),
        "dprice/ds0": disc * np.mean(itm * st / m.s0),
        "dprice/dvol": disc * np.mean(itm * st * (math.sqrt(dt) * zsum - m.vol * m.maturity)),
    }


def check_pathwise(o, zsum, steps, tol):
    for name, w in pathwise(zsum, steps).items():
        v = float(np.asarray(o[name]).reshape(-1)[0])
        assert abs(v - w) <= tol * (1 + abs(w)), (name, v, w)
    cf = bs.analytic()
    assert abs(float(o["dprice/ds0"]) - cf["delta"]) <= 0.02
    assert abs(float(o["dprice/dvol"]) - cf["vega"]) <= 1.5


def test_config5_greeks_f64_full_size_pathwise(device):
    """The benchmark's f64 graph at 2^22 paths x 64 steps (its gather
    adjoint, a scatter into 2^28 bins through the strided index p*64 + 63,
    is computed where the adjoint map reads it) against the pathwise estimator on the same
    Philox draws, within 1e-9 relative (summation order is the only
    difference)."""
    n, steps = C.PATHS5, C.STEPS5
    g = C.mc_greeks(n, steps, F64)
    assert "scan_rowseq" in roles(g) and not {"scatter_affine", "reduce_rowseq"} & set(roles(g))
    o = run_dev(g, bs.inputs(F64, seed=7))
    zg = Graph.create("z", [("z", rng.normal(F64, D.scalar("seed", I32), (n, steps)))])
    z = run_dev(zg, [("seed", np.array(7, np.int32))])["z"]
    assert np.isfinite(z).all()
    zsum = z.sum(axis=1, dtype=np.float64)
    del z
    check_pathwise(o, zsum, steps, 1e-9)


def nonfinite_class(v):
    v = np.asarray(v, dtype=np.float64)
    return np.where(np.isnan(v), 3, np.where(np.isposinf(v), 1, np.where(np.isneginf(v), 2, 0)))


@pytest.mark.parametrize("plant", ["+inf", "-inf", "both"])
def test_config5_greeks_f32_infinite_draws_vs_oracle(device, plant):
    """Infinite normal draws through the f32 path pricer and its adjoint,
    on the device and on the oracle: the same inf/NaN in the same outputs
    (the interpreter's semantics: one +inf draw makes the price +inf and
    delta NaN; any infinite draw makes vega NaN through the scan adjoint's
    total - prefix + abar), every finite output within the band."""
    n, steps = 4096, C.STEPS5
    g = bs.call_paths_greeks(n, steps, F32, draws=D.param("z", F32, (n, steps)))
    z = C.normals(11, (n, steps), F32)
    if plant in ("+inf", "both"):
        z[17, 5] = np.inf
    if plant in ("-inf", "both"):
        z[100, 63] = -np.inf
    ins = [x for x in bs.inputs(F32) if x[0] != "seed"] + [("z", z)]
    exp = dict(oracle.run(g, ins))
    got = run_dev(g, ins)
    for name, e in exp.items():
        np.testing.assert_array_equal(nonfinite_class(got[name]), nonfinite_class(e), err_msg=name)
        fin = np.isfinite(np.asarray(e, dtype=np.float64))
        assert band(np.asarray(got[name])[fin], np.asarray(e)[fin], 1e-4) <= 1e-4, name
    assert np.isnan(got["dprice/dvol"])
    assert bool(np.isposinf(got["price"])) == (plant != "-inf")


def test_config5_greeks_f32_full_size(device):
    """Config 5 in f32 at 2^22 paths x 64 steps. The reference's generator
    computes u = (w + 0.5) 2^-32 in f64 and casts it to f32
    (rng.ml:61-67), then 2u - 1 in f32 (rng.ml:69-71): the 128 largest
    words give u = 1 and the 64 smallest 2u - 1 = -1, so z = +-inf with
    probability 3 * 2^-26 per draw, about 12 of the 2^28 draws. So:
    (1) the device's non-finite draws are exactly those words (from the
    bit-exact Philox stream), with the signs the f32 rounding gives;
    (2) the benchmark's graph returns what the interpreter returns for such
    draws: price +inf, delta and vega NaN;
    (3) the same graph with finite draws (a param: the f64 normals cast to
    f32) checks the f32 adjoint at full size: price, delta and vega
    against the pathwise estimator on those draws, within the
    accumulation band 1e-4."""
    n, steps = C.PATHS5, C.STEPS5
    wg = Graph.create("w", [("w", rng.u32(D.scalar("seed", I32), (n, steps)))])
    w = run_dev(wg, [("seed", np.array(7, np.int32))])["w"].view(np.uint32).reshape(-1)
    # the interpreter's rounding (R1): u to f32, 2u rounded, then - 1 rounded
    u = ((w.astype(np.float64) + 0.5) * 2.0 ** -32).astype(np.float32)
    t = ((2.0 * u.astype(np.float64)).astype(np.float32).astype(np.float64) - 1.0).astype(np.float32)
    del u, w
    zg = Graph.create("z", [("z", rng.normal(F32, D.scalar("seed", I32), (n, steps)))])
    z = run_dev(zg, [("seed", np.array(7, np.int32))])["z"].reshape(-1)
    np.testing.assert_array_equal(np.flatnonzero(np.isposinf(z)), np.flatnonzero(t == 1.0))
    np.testing.assert_array_equal(np.flatnonzero(np.isneginf(z)), np.flatnonzero(t == -1.0))
    assert not np.isnan(z).any() and (t == 1.0).any() and (t == -1.0).any()
    del z, t
    o = run_dev(C.mc_greeks(n, steps, F32), bs.inputs(F32, seed=7))
    assert np.isposinf(o["price"]) and np.isnan(o["dprice/ds0"]) and np.isnan(o["dprice/dvol"])
    zf = gen(C.gen_normals((n, steps), F32), 7)
    assert np.isfinite(zf).all()
    g = bs.call_paths_greeks(n, steps, F32, draws=D.param("z", F32, (n, steps)))
    assert "scan_rowseq" in roles(g) and not {"scatter_affine", "reduce_rowseq"} & set(roles(g))
    o = run_dev(g, [x for x in bs.inputs(F32) if x[0] != "seed"] + [("z", zf)])
    zsum = zf.sum(axis=1, dtype=np.float64)
    del zf
    check_pathwise(o, zsum, steps, 1e-4)


@pytest.mark.parametrize("tune,tpl", [("", {"scatter_affine"}),
                                      ("scatter_affine=0", {"scatter_coarse", "scatter_windows"}),
                                      ("scatter_affine=0,scatter_lds=0", {"scatter_zero", "scatter_atomic"})])
def test_gather_adjoint_of_the_last_column(device, monkeypatch, tune, tpl):
    """The adjoint of picking the last column of an f32[2^20 + 8; 64] by a
    gather, as the path pricer does: a scatter_add into 2^26 + 512 bins
    through the index p*64 + 63, one pass over the bins by default (the
    index is affine and in range, so each bin takes at most one value);
    with scatter_affine=0, the two-level LDS path over 4097 slices; with
    scatter_lds=0 as well, scatter_zero + scatter_atomic; against the
    oracle."""
    monkeypatch.setenv("CCHIP_TUNE", tune)
    rows, steps = (1 << 20) + 8, 64
    x = D.param("x", F32, (rows, steps))
    idx = D.map(lambda p: D.add(D.mul(p, D.const(I32, steps)), D.const(I32, steps - 1)), D.iota((rows,)))
    st = D.gather(idx, x)
    payoff = D.map(lambda s: D.mul(s, D.max(D.sub(s, D.const(F32, 0.25)), D.const(F32, 0.0))), st)
    loss = D.reduce(D.add, D.const(F32, 0.0), payoff)
    g = G.grad(Graph.create("pick", [("loss", loss)]), "loss", ["x"])
    assert tpl <= set(roles(g))
    xv = np.random.default_rng(3).uniform(-1, 1, (rows, steps)).astype(np.float32)
    exp = oracle.run(g, [("x", xv)])
    got = run_dev(g, [("x", xv)])
    bad = [v for v in Diff.policy_check(g, exp, list(got.items())) if not v.ok]
    assert not bad, bad
    dx = got["dloss/dx"]
    assert np.count_nonzero(dx[:, :-1]) == 0 and np.count_nonzero(dx[:, -1]) > rows // 3
