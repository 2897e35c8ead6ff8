"""Longstaff-Schwartz on the CPU oracle, as the reference tests it on its
interpreter (test/unit/test_lsm.ml:23-49): the host references, the price
band against the binomial tree, determinism per seed, and three compiles
that the pricing loop never repeats. No GPU."""

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd.examples import lsm


def test_references():
    assert abs(lsm.binomial_american_put(500) - 6.09) <= 0.02
    assert abs(lsm.european_put() - 5.5735) <= 1e-3


def test_solve3():
    x = lsm.solve3([[2.0, 1.0, 0.0], [1.0, 3.0, 1.0], [0.0, 1.0, 4.0]], [3.0, 5.0, 5.0])
    assert max(abs(a - b) for a, b in zip(x, [1.0, 1.0, 1.0])) < 1e-12
    assert lsm.solve3([[1.0, 2.0, 3.0], [2.0, 4.0, 6.0], [0.0, 0.0, 0.0]], [1.0, 2.0, 3.0]) == [0.0, 0.0, 0.0]


def test_price_within_band_of_binomial():
    binom, euro = lsm.binomial_american_put(500), lsm.european_put()
    px = lsm.Make(oracle.Interp, 8192, 50).price(11)
    assert abs(px - binom) <= 0.25
    assert px >= euro - 0.05


def test_deterministic_per_seed():
    t = lsm.Make(oracle.Interp, 4096, 20)
    a, b, c = t.price(11), t.price(11), t.price(12)
    assert a == b
    assert abs(a - c) < 0.5


class Counting:
    name = "counting-interp"
    compiles = 0

    @classmethod
    def compile(cls, g):
        cls.compiles += 1
        return oracle.Interp.compile(g)

    run = staticmethod(oracle.Interp.run)


def test_three_compiles():
    Counting.compiles = 0
    t = lsm.Make(Counting, 256, 4)
    assert Counting.compiles == 3
    t.price(1)
    assert Counting.compiles == 3


def test_regression_products_split_k():
    """X^T X and X^T y ([3;n] x [n;3], [3;n] x [n;1]) take the split-k
    template; the [n;3] x [3;1] fitted continuation keeps the tiling."""
    def roles(g):
        return [l.split()[2] for l in H.plan(g).splitlines() if l.startswith("kernel")]

    r = roles(lsm.regress_graph(65536, 50, 100.0, 0.999))
    assert r.count("matmul_splitk") == 2 and r.count("matmul_ksum") == 2
    assert "matmul_tiled" in roles(lsm.update_graph(65536, 50, 100.0, 0.999))
