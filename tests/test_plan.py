"""Structure of what Backend_hip generates, read off its plan and source
without a device: the fusion plan (Fusion.plan's four rules,
fusion.ml:41-73), kernel counts and template choice per root, the host
plan's shape (lower.ml:968-1012), the printer's integer-exactness
spellings, and that generated modules compile for gfx950 with hiprtc.
Mirrors test_fusion.ml, test_lower.ml, test_multikernel.ml, test_emit.ml,
test_scatter.ml:50-70 and test_matmul.ml:105-139."""

import numpy as np
import pytest

from cudacaml_amd import backend_hip as H
from cudacaml_amd import dsl as D
from cudacaml_amd import rng
from cudacaml_amd import runtime
from cudacaml_amd.examples import configs as C
from cudacaml_amd.examples import programs as P
from cudacaml_amd.examples import saxpy as sx
from cudacaml_amd.ir import F32, F64, I32, I64, Graph


def parse(plan):
    bufs, kernels, ops = [], [], []
    for line in plan.splitlines():
        f = line.split()
        if f[0] == "buffer":
            bufs.append((f[2], f[3], int(f[4]), f[5]))
        elif f[0] == "kernel":
            kernels.append((f[1], f[2]))
        elif f[0] in ("alloc", "upload", "launch", "download", "free"):
            ops.append(tuple(f))
    return bufs, kernels, ops


def kernels_of(g):
    return parse(H.plan(g))[1]


def test_chain_is_one_kernel():
    assert [t for _, t in kernels_of(P.chain(4096).graph())] == ["map"]


def test_saxpy_is_map_then_reduce(monkeypatch):
    """s = sum(r) of the map's own output folds inside the map kernel (one
    partial a workgroup, then the fold); fuse_reduce=0 keeps the split
    reduction that reads r back."""
    ks = kernels_of(sx.program(1 << 18, 2.0))
    assert [t for _, t in ks] == ["map", "reduce_split_fold"]
    bufs, kk, _ = parse(H.plan(sx.program(1 << 18, 2.0)))
    part = [b for b in bufs if b[0].endswith("_partials")]
    assert len(part) == 1 and part[0][3] == "scratch" and part[0][2] == 4 * 256  # one a wave
    # 2^20: 4096 partials, folded by one workgroup of 1024 threads;
    # fold_one=0, or 2^24 (65536 partials): 1024 a workgroup, then a
    # second kernel
    assert [t for _, t in kernels_of(sx.program(1 << 20, 2.0))] == ["map", "reduce_split_fold"]
    fold = [f.split() for f in H.plan(sx.program(1 << 20, 2.0)).splitlines() if "reduce_split_fold" in f]
    assert fold[0][fold[0].index("grid") + 1] == "1" and fold[0][fold[0].index("block") + 1] == "1024"
    assert [t for _, t in kernels_of(sx.program(1 << 24, 2.0))] == ["map", "reduce_split_fold", "reduce_split_fold"]
    monkeypatch.setenv("CCHIP_TUNE", "fold_one=0")
    assert [t for _, t in kernels_of(sx.program(1 << 20, 2.0))] == ["map", "reduce_split_fold", "reduce_split_fold"]
    monkeypatch.setenv("CCHIP_TUNE", "fuse_reduce=0")
    ks = kernels_of(sx.program(1 << 20, 2.0))
    assert [t for _, t in ks] == ["map", "reduce_split", "reduce_split_fold"]


def test_reduction_of_an_expression_folds_in_its_producer(monkeypatch):
    """sum(a * z) beside the map that makes a folds inside that map's
    kernel, which also loads z; so does an expression of a 2-D map read
    flattened, of a gather root's output, and one with another root in
    between. Not when the expression reads the map's output at another
    index, or when fuse_reduce_expr=0."""
    n = 1 << 18
    x, y, z = (D.param(c, F32, (n,)) for c in "xyz")
    z0 = D.const(F32, 0.0)
    a = D.map2(D.add, x, y)
    g = Graph.create("e", [("a", a), ("s", D.reduce(D.add, z0, D.map2(D.mul, a, z)))])
    assert [t for _, t in kernels_of(g)] == ["map", "reduce_split_fold"]
    moved = _bytes(g, "moved")
    assert moved["map"] == 3 * 4 * n + 4 * n  # x, y, a, and z for the expression
    # a root in between, reading the sum's other input
    u = D.map(lambda v: D.mul(v, v), z)
    g = Graph.create("e", [("a", a), ("u", u), ("s", D.reduce(D.max, z0, D.map2(D.mul, a, z)))])
    assert [t for _, t in kernels_of(g)] == ["map", "map", "reduce_split_fold"]
    # 2-D, flattened
    x2, w2 = D.param("x2", F32, (64, 4096)), D.param("w2", F32, (64, 4096))
    a2 = D.map(lambda v: D.add(v, v), x2)
    g = Graph.create("e", [("a", a2), ("s", D.reduce(D.add, z0, D.flatten(D.map2(D.mul, a2, w2))))])
    assert [t for _, t in kernels_of(g)] == ["map", "reduce_split_fold"]
    # a gather root
    idx = D.param("idx", I32, (n,))
    st = D.map(D.exp, D.gather(idx, x))
    g = Graph.create("e", [("st", st), ("s", D.reduce(D.add, z0, D.map(lambda v: D.max(v, z0), st)))])
    assert "reduce_split" not in [t for _, t in kernels_of(g)]
    # the map's output read at another index: its own split reduction
    rev = D.map(lambda i: D.sub(D.const(I32, n - 1), i), D.iota((n,)))
    g = Graph.create("e", [("a", a), ("s", D.reduce(D.add, z0, D.map2(D.mul, D.gather(rev, a), z)))])
    assert "reduce_split" in [t for _, t in kernels_of(g)]
    # a read only by the expression (twice, so materialised): its kernel
    # stores nothing but the partials, and its buffer is elided
    g = Graph.create("e", [("s", D.reduce(D.add, z0, D.map2(D.add, D.map2(D.mul, a, z), a)))])
    bufs, ks, _ = parse(H.plan(g))
    assert [t for _, t in ks] == ["map", "reduce_split_fold"]
    assert [b[3] for b in bufs if b[2] == n] == ["param", "param", "param", "elided"]
    assert _bytes(g, "moved")["map"] == 3 * 4 * n
    monkeypatch.setenv("CCHIP_TUNE", "skip_unread_stores=0")
    assert [b[3] for b in parse(H.plan(g))[0] if b[2] == n] == ["param", "param", "param", "computed"]
    monkeypatch.setenv("CCHIP_TUNE", "fuse_reduce_expr=0")
    g = Graph.create("e", [("a", a), ("s", D.reduce(D.add, z0, D.map2(D.mul, a, z)))])
    assert [t for _, t in kernels_of(g)] == ["map", "reduce_split", "reduce_split_fold"]
    monkeypatch.delenv("CCHIP_TUNE")
    # config 5's adjoint sums and its price: no split reduction left
    assert "reduce_split" not in [t for _, t in kernels_of(C.mc_greeks())]


def test_affine_scatter_is_read_in_place(monkeypatch):
    """A scatter_add whose index is a*j + b, injective and in range, is
    computed where it is read (0 + its one source value, or 0): no scatter
    kernel, its buffer elided. It keeps both when it is an output, and with
    scatter_inline=0; an index that can leave the range is never read in
    place."""
    n = 1 << 16
    src, y = D.param("src", F32, (n,)), D.param("y", F32, (64 * n,))
    idx = D.map(lambda p: D.add(D.mul(p, D.const(I32, 64)), D.const(I32, 63)), D.iota((n,)))
    h = D.scatter_add(idx, D.map(lambda v: D.mul(v, v), src), (64 * n,))
    o = D.map2(D.mul, h, y)
    g = Graph.create("s", [("o", o)])
    bufs, ks, _ = parse(H.plan(g))
    assert [t for _, t in ks] == ["map"]
    assert [b[3] for b in bufs if b[2] == 64 * n] == ["param", "elided", "computed"]
    assert [t for _, t in kernels_of(Graph.create("s", [("o", o), ("h", h)]))] == ["scatter_affine", "map"]
    # a matmul operand computes it too, as its element function
    w = D.param("w", F32, (64, 16))
    assert [t for _, t in kernels_of(Graph.create("m", [("c", D.matmul(D.reshape((n, 64), h), w))]))] == ["matmul_tiled"]
    wide = D.map(lambda p: D.mul(p, D.const(I32, 65)), D.iota((n,)))
    g = Graph.create("s", [("o", D.map2(D.mul, D.scatter_add(wide, src, (64 * n,)), y))])
    assert "map" in [t for _, t in kernels_of(g)] and len(kernels_of(g)) > 1
    monkeypatch.setenv("CCHIP_TUNE", "scatter_inline=0")
    assert [t for _, t in kernels_of(Graph.create("s", [("o", o)]))] == ["scatter_affine", "map"]
    monkeypatch.delenv("CCHIP_TUNE")
    # config 5's gather adjoint
    assert "scatter_affine" not in [t for _, t in kernels_of(C.mc_greeks())]


def test_two_groups_a_lane_for_exp_maps_with_varying_loads(monkeypatch):
    """An f32 map that calls exp and gathers at varying indices takes two
    16-byte groups a lane; one that calls exp but only streams, or only
    gathers, keeps one; map_unroll_gx=0 keeps one everywhere."""
    n = 1 << 18
    x, y, gi = D.param("x", F32, (n,)), D.param("y", F32, (n,)), D.param("gi", I32, (n,))

    def groups(g):
        src = H.source(g)
        k = src[src.index("void k_"):]
        return 2 if "cc_v4<float> r[2];" in k else 1 if "cc_v4<float> r;" in k else 0

    both = Graph.create("eg", [("o", D.map2(lambda u, v: D.mul(D.exp(u), v), x, D.gather(gi, y)))])
    stream = Graph.create("e", [("o", D.map2(lambda u, v: D.mul(D.exp(u), v), x, y))])
    gather = Graph.create("g", [("o", D.map2(D.mul, x, D.gather(gi, y)))])
    assert (groups(both), groups(stream), groups(gather)) == (2, 1, 1)
    monkeypatch.setenv("CCHIP_TUNE", "map_unroll_gx=0")
    assert groups(both) == 1


def test_fanout_materialises_shared_node_once():
    bufs, ks, _ = parse(H.plan(P.fanout(1000).graph()))
    computed = [b for b in bufs if b[3] == "computed"]
    # s = x*x (fan-out 3) plus the three outputs a, b, c
    assert len(computed) == 4 and len(ks) == 4


def test_transpose_fuses_into_rows_reduce():
    x = D.param("x", F32, (8, 16))
    r = D.reduce_rows(D.add, D.const(F32, 0.0), D.map(lambda e: D.mul(e, e), D.transpose(x)))
    bufs, ks, _ = parse(H.plan(Graph.create("g", [("r", r)])))
    assert len(ks) == 1 and [b[3] for b in bufs] == ["param", "computed"]


def test_barriers_are_materialised():
    idx, src = D.param("idx", I32, (6,)), D.param("src", F32, (6,))
    s = D.scatter_add(idx, src, (4,))
    bufs, ks, ops = parse(H.plan(Graph.create("h", [("r", D.map(D.neg, s))])))
    assert [t for _, t in ks] == ["scatter_direct", "map"]
    launches = [o[1] for o in ops if o[0] == "launch"]
    assert launches == [k for k, _ in ks]


def test_scatter_template_choice(monkeypatch):
    """One slice (16384 bins by default, 8192 for 8-byte types): direct LDS
    fold; up to 256 slices: a partition into tile-local runs, no count or
    offset passes; more (or scatter_local_max=0): per-chunk counts, offsets,
    then the partition; tables too large for the slice limit (or
    scatter_lds=0): global atomics."""
    def ks(n, bins, dt=F32):
        i, s = D.param("i", I32, (n,)), D.param("s", dt, (n,))
        return [t for _, t in kernels_of(Graph.create("h", [("h", D.scatter_add(i, s, (bins,)))]))]

    assert ks(1000, 8192) == ["scatter_direct"]
    assert ks(100000, 16384) == ["scatter_direct", "scatter_reduce"]
    assert ks(100000, 8193, F64) == ["scatter_partition", "scatter_accumulate", "scatter_reduce"]
    assert ks(100000, 16385) == ["scatter_partition", "scatter_accumulate", "scatter_reduce"]
    assert ks(1 << 22, 256 * 16384) == ["scatter_partition", "scatter_accumulate", "scatter_reduce"]
    assert ks(1 << 22, 256 * 16384 + 1)[:4] == ["scatter_count", "scatter_colscan", "scatter_bscan", "scatter_partition"]
    assert ks(1 << 22, 1 << 28) == ["scatter_zero", "scatter_atomic"]
    # two levels in windows up to 8192 slices (128 super-slices)
    assert "scatter_windows" in ks(1 << 20, 8192 * 16384) and ks(1 << 20, 8192 * 16384 + 1)[-1] == "scatter_atomic"
    monkeypatch.setenv("CCHIP_TUNE", "scatter_local_max=0")
    assert ks(100000, 16385)[:4] == ["scatter_count", "scatter_colscan", "scatter_bscan", "scatter_partition"]
    monkeypatch.setenv("CCHIP_TUNE", "scatter_lds=0")
    assert ks(1000, 4096) == ["scatter_zero", "scatter_atomic"]


def test_matmul_barrier_fuses_operand_maps():
    a, b = D.param("a", F64, (20, 30)), D.param("b", F64, (30, 10))
    bufs, ks, _ = parse(H.plan(Graph.create("mm", [("c", D.matmul(D.map(D.exp, a), b))])))
    assert len(ks) == 1 and ks[0][1].startswith("matmul")
    assert [b[0] for b in bufs] == ["p_a", "p_b", bufs[2][0]]


def test_host_plan_shape():
    """Alloc params then computed, upload, launches, download, free in the
    same order as alloc (lower.ml:977-1011)."""
    bufs, ks, ops = parse(H.plan(sx.program(1024, 2.0)))
    kinds = [o[0] for o in ops]
    first_upload = kinds.index("upload")
    assert all(k == "alloc" for k in kinds[:first_upload])
    assert kinds[first_upload:first_upload + 2] == ["upload", "upload"]
    assert [o[1] for o in ops if o[0] == "download"] == ["r", "s"]
    allocs = [o[1] for o in ops if o[0] == "alloc"]
    frees = [o[1] for o in ops if o[0] == "free"]
    assert sorted(allocs) == sorted(frees)


def test_uniform_graph_uploads_only_the_seed():
    g = Graph.create("u", [("r", rng.uniform(F32, D.scalar("seed", I32), (16,)))])
    _, _, ops = parse(H.plan(g))
    assert [o for o in ops if o[0] == "upload"] == [("upload", "seed", "p_seed")]


@pytest.mark.parametrize("rows,n,tpl", [(8192, 8192, "reduce_block"), (8192, 1023, "reduce_rowseq"),
                                        (8192, 1024, "reduce_wave"), (1, 1 << 24, "reduce_split"),
                                        (600, 4096, "reduce_block"), (64, 64, "reduce_wave")])
def test_reduce_template_choice(rows, n, tpl):
    x = D.param("x", F32, (rows, n))
    got = [t for _, t in kernels_of(Graph.create("r", [("s", D.reduce_rows(D.add, D.const(F32, 0), x))]))]
    assert got == ([tpl, "reduce_split_fold"] if tpl == "reduce_split" else [tpl])


@pytest.mark.parametrize("rows,n,tpls", [(8192, 8192, ["scan_tile"]), (8192, 2047, ["scan_rowseq"]),
                                         (1024, 40000, ["scan_init", "scan_lookback"]), (1, 1 << 28, ["scan_init", "scan_lookback"]),
                                         (100, 5000, ["scan_tile"]), (100, 50, ["scan_wave"])])
def test_scan_template_choice(rows, n, tpls):
    x = D.param("x", I32, (rows, n))
    assert [t for _, t in kernels_of(Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 0), x))]))] == tpls


def test_config_plans():
    # rows of 8192 fold as trees, a workgroup a row (the adds within the
    # rounding of another grouping, the max bit-exact), all three roots in
    # one kernel that reads each row once
    assert [t for _, t in kernels_of(C.rows())] == ["scan_tile_fold"]
    # the gather back reads the scatter's partition: the table slice by
    # slice from LDS, then each tile's values back in element order; 128
    # slices, so the partition keeps each tile's pairs in the tile's region
    assert [t for _, t in kernels_of(C.scatter_gather())] == ["scatter_partition", "scatter_accumulate",
                                                               "scatter_reduce", "gather_slices", "gather_unpartition"]
    # 2^26 bins: one workgroup per slice stores its table, no partials, and
    # puts h[key] in the pairs itself (no slice kernel); two partition
    # levels, the slice pass in windows of each super-slice's run, undone
    # level by level
    perm = [t for _, t in kernels_of(C.scatter_gather(C.N3, C.N3))]
    assert perm == ["scatter_count", "scatter_colscan", "scatter_bscan", "scatter_coarse", "scatter_windows",
                    "scatter_partition", "scatter_accumulate", "gather_unpartition", "gather_unpartition"]


def test_gather_back_only_over_the_same_index(monkeypatch):
    """A gather root reads back through the scatter's partition only when
    its index is the scatter's own index tensor and the partition is staged;
    scatter_gather_back=0 keeps the plain gather."""
    n, bins = 1 << 20, 1 << 16
    idx, idx2 = D.param("idx", I32, (n,)), D.param("idx2", I32, (n,))
    src = D.param("src", F32, (n,))
    h = D.scatter_add(idx, src, (bins,))
    roles = lambda g: [t for _, t in kernels_of(g)]  # noqa: E731
    assert roles(Graph.create("a", [("h", h), ("b", D.gather(idx, h))]))[-2:] == ["gather_slices", "gather_unpartition"]
    assert roles(Graph.create("a", [("h", h), ("b", D.gather(idx2, h))]))[-1] == "map"
    # one slice (no partition): the plain gather
    small = D.scatter_add(idx, src, (4096,))
    assert roles(Graph.create("a", [("h", small), ("b", D.gather(idx, small))]))[-1] == "map"
    monkeypatch.setenv("CCHIP_TUNE", "scatter_gather_back=0")
    assert roles(Graph.create("a", [("h", h), ("b", D.gather(idx, h))]))[-1] == "map"
    # the partition's buffers live until the gather back has run
    monkeypatch.delenv("CCHIP_TUNE")
    plan = H.plan(Graph.create("a", [("h", h), ("b", D.gather(idx, h))])).splitlines()
    last_launch = max(i for i, l in enumerate(plan) if l.startswith("launch"))
    frees = [l.split()[1] for l in plan[last_launch:] if l.startswith("free")]
    assert any(b.endswith("_slot") for b in frees) and any(b.endswith("_val") for b in frees)
    ks = kernels_of(C.mc_paths())
    assert "scan_rowseq" in [t for _, t in ks]


def test_printer_integer_exactness():
    """Wrapping through unsigned, masked logical shifts, OCaml min/max and
    the f32-constant rule (emit.ml:60-135 and cudacaml_backend_interp.ml
    :246)."""
    x = D.param("x", I32, (4,))
    src = H.source(Graph.create("g", [("r", D.map(lambda e: D.shr(D.mul(e, D.const(I32, 3)), D.const(I32, 3)), x))]))
    assert "(cc_u32)" in src and "& 31" in src
    y = D.param("y", I64, (4,))
    src = H.source(Graph.create("g", [("r", D.map(lambda e: D.shl(e, D.const(I64, 3)), y))]))
    assert "cc_u64" in src and "& 63" in src
    z = D.param("z", F32, (4,))
    src = H.source(Graph.create("g", [("r", D.map(lambda e: D.max(D.mul(e, D.const(F32, 0.1)), e), z))]))
    assert "(float)(" in src and "(double)" in src and "cc_maxf" in src
    # erfinv is the backend's own: cc_erfinvf in f32, cc_erfinv in f64 (the
    # element functions follow the shared prelude)
    src = H.source(Graph.create("g", [("r", D.map(lambda e: D.erfinv(D.sin(e)), z))]))
    body = src[src.rindex("__device__ __forceinline__ float f_"):]
    assert "cc_erfinvf(" in body and "sinf(" in body
    w = D.param("w", F64, (4,))
    src = H.source(Graph.create("g", [("r", D.map(lambda e: D.erfinv(D.cos(e)), w))]))
    body = src[src.rindex("__device__ __forceinline__ double f_"):]
    assert "cc_erfinv(" in body and "erfinvf(" not in body


def test_generated_modules_compile_for_gfx950():
    for g in [C.rows(2048, 1024), C.global_scan(1 << 16), C.scatter_gather(1 << 12, 1 << 8),
              C.matmul(64), C.mc_paths(256, 16), P.bs_greeks(1024).graph()]:
        assert runtime.Jit.check(g.name, H.source(g)) > 0


def test_jit_reports_compile_errors():
    with pytest.raises(RuntimeError, match="hiprtc"):
        runtime.Jit.check("bad", "this is not HIP")


def _bytes(g, field="bytes"):
    return {k[2]: int(k[k.index(field) + 1]) for k in
            (l.split() for l in H.plan(g).splitlines() if l.startswith("kernel"))}


def test_algorithmic_bytes_per_kernel(monkeypatch):
    """Each root's algorithmic bytes sit on its main kernel: identity reads
    count the elements read, a gather one element per output, a broadcast
    source one; helper kernels carry none. A reduction folded inside its
    input's map keeps its root's bytes (its input read once), on its last
    fold."""
    n = 1 << 20
    b = _bytes(sx.program(n, 2.0))
    assert b["map"] == 3 * 4 * n and b["reduce_split_fold"] == 4 * n + 4
    # ... but reads nothing back: it moves its one output value
    m = _bytes(sx.program(n, 2.0), "moved")
    assert m["map"] == 3 * 4 * n and m["reduce_split_fold"] == 4
    monkeypatch.setenv("CCHIP_TUNE", "fuse_reduce=0")
    b = _bytes(sx.program(n, 2.0))
    assert b["map"] == 3 * 4 * n and b["reduce_split"] == 4 * n + 4
    assert _bytes(sx.program(n, 2.0), "moved") == b
    monkeypatch.delenv("CCHIP_TUNE")
    b = _bytes(C.global_scan(n))
    assert b["scan_lookback"] == 8 * n and b["scan_init"] == 0
    b = _bytes(C.scatter_gather(n, 1 << 15))
    assert b["scatter_partition"] == 8 * n + 4 * (1 << 15)
    assert b["scatter_accumulate"] == 0 and b["scatter_reduce"] == 0
    # the gather back: idx, the table (once), out, on its last kernel
    assert b["gather_unpartition"] == 4 * n + 4 * (1 << 15) + 4 * n and b["gather_slices"] == 0
    # the price reduces the gathered last column only, not the whole path matrix
    b = _bytes(C.mc_paths(4096, 64))
    assert b["reduce_split"] < 4 * 4096 + 64


def test_sibling_row_roots_share_one_kernel(monkeypatch):
    """A row scan taking the one-tile-a-row template and the tree-folded
    reductions of the same tensor's rows are one kernel: it carries every
    root's algorithmic bytes and moves the tensor once plus the outputs.
    Reductions of another tensor, or of the same one in order, keep their
    own kernels; sibling_fuse=0 keeps every root its own."""
    n = C.ROWS2
    b, m = _bytes(C.rows()), _bytes(C.rows(), "moved")
    assert b == {"scan_tile_fold": 3 * 4 * n * n + 4 * n * n + 2 * 4 * n}
    assert m == {"scan_tile_fold": 4 * n * n + 4 * n * n + 2 * 4 * n}
    x, y = D.param("x", F32, (600, 3000)), D.param("y", F32, (600, 3000))
    g = Graph.create("g", [("a", D.reduce_rows(D.add, D.const(F32, 0.0), y)),
                           ("p", D.scan_rows(D.add, D.const(F32, 0.0), x)),
                           ("b", D.reduce_rows(D.max, D.const(F32, 0.0), x)),
                           ("c", D.reduce(D.add, D.const(F32, 0.0), x))])
    assert [t for _, t in kernels_of(g)] == ["reduce_block", "scan_tile_fold", "reduce_split", "reduce_split_fold"]
    monkeypatch.setenv("CCHIP_TUNE", "sibling_fuse=0,same_fold=0")
    assert [t for _, t in kernels_of(C.rows())] == ["reduce_block", "reduce_block", "scan_tile"]
    # in order (the interpreter's exact folds): nothing to share
    monkeypatch.setenv("CCHIP_TUNE", "rr_tree=1,rs_tree=0,same_fold=0")
    assert [t for _, t in kernels_of(C.rows())] == ["reduce_rowseq", "reduce_block", "scan_rowseq"]
    # a look-back scan (several tiles a row) keeps the reductions apart
    monkeypatch.delenv("CCHIP_TUNE")
    z = D.param("z", I32, (4, 100000))
    g = Graph.create("lb", [("p", D.scan_rows(D.add, D.const(I32, 0), z)),
                            ("s", D.reduce_rows(D.max, D.const(I32, 0), z))])
    assert "scan_tile_fold" not in [t for _, t in kernels_of(g)]


def _kernel_args(g):
    """(template, [buffer names]) of every kernel, in launch order."""
    lines = [l.split() for l in H.plan(g).splitlines()]
    names = {f[1]: f[2] for f in lines if f[0] == "buffer"}
    return [(f[2], [names[a] for a in f[f.index("args") + 1:]]) for f in lines if f[0] == "kernel"]


SAME_FOLD_SHAPES = [
    ((100, 50), F32, "scan_wave", ""),
    ((600, 3000), F32, "scan_tile", ""),
    ((4, 100000), I32, "scan_lookback", ""),
    ((2048, 300), F32, "scan_rowseq", ""),
    ((1024, 40000), F32, "scan_rowseq", "rs_tree=0"),  # split roles
    ((1 << 20,), F64, "scan_lookback", ""),
]


@pytest.mark.parametrize("shape,dt,template,knobs", SAME_FOLD_SHAPES)
def test_same_fold_reduction_reads_the_scans_row_ends(monkeypatch, shape, dt, template, knobs):
    """A reduction with the scan's own combine and init over the same
    tensor launches nothing: whichever template the scan takes stores each
    row's last element into the reduction's buffer. Another init, another
    combine or same_fold=0 keeps the reduction's own kernels."""
    monkeypatch.setenv("CCHIP_TUNE", knobs)
    x = D.param("x", dt, shape)
    z = D.const(dt, 0 if dt is I32 else 0.0)

    def graph(init, comb=D.add):
        return Graph.create("sf", [("s", D.scan(D.add, z, x) if len(shape) == 1 else D.scan_rows(D.add, z, x)),
                                   ("r", D.reduce(comb, init, x) if len(shape) == 1 else D.reduce_rows(comb, init, x))])

    g = graph(z)
    main = [k for k in _kernel_args(g) if k[0] != "scan_init"]
    assert [t for t, _ in main] == [template]
    bufs = {n: l.split()[2] for l in H.plan(g).splitlines() for n in ["s", "r"]
            if l.startswith("download " + n + " ")}
    assert bufs["r"] in main[0][1] and bufs["s"] in main[0][1]
    # otherwise its own kernels, or a tree sibling of a one-tile-a-row scan
    def templates(g):
        return [t for t, _ in _kernel_args(g) if t != "scan_init"]
    one = D.const(dt, 1 if dt is I32 else 1.0)
    assert templates(graph(one)) != [template]
    assert templates(graph(z, D.max)) != [template]
    monkeypatch.setenv("CCHIP_TUNE", ",".join(k for k in [knobs, "same_fold=0"] if k))
    assert templates(graph(z)) != [template]


def test_same_fold_runs_at_the_reductions_place():
    """A same-fold pair whose reduction comes first in the plan, with a root
    reading the reduction in between: the scan's kernel runs at the
    reduction's place, so the reader runs after it. Monte Carlo greeks lose
    their row reduction of the adjoint (total - prefix + adjoint)."""
    x = D.param("x", F32, (2048, 300))
    z = D.const(F32, 0.0)
    r = D.reduce_rows(D.add, z, x)
    m = D.map(lambda v: D.mul(v, D.const(F32, 2.0)), r)
    s = D.scan_rows(D.add, z, x)
    g = Graph.create("sf", [("m", m), ("s", s)])
    assert [t for t, _ in _kernel_args(g)] == ["scan_rowseq", "map"]
    assert "reduce_rowseq" not in [t for _, t in kernels_of(C.mc_greeks())]


def _launch_uses_live_buffers(g):
    """Every buffer a launched kernel takes is allocated before the launch
    and freed only after the last launch that takes it."""
    lines = [l.split() for l in H.plan(g).splitlines()]
    names = {}
    kargs = {}
    for f in lines:
        if f[0] == "buffer":
            names[f[1]] = f[2]
        elif f[0] == "kernel":
            kargs[f[1]] = [names[a] for a in f[f.index("args") + 1:]]
    live = set()
    for f in lines:
        if f[0] == "alloc":
            live.add(f[1])
        elif f[0] == "free":
            live.discard(f[1])
        elif f[0] == "launch":
            dead = [b for b in kargs[f[1]] if b not in live and b != "err"]
            assert not dead, (g.name, f[1], dead)


@pytest.mark.parametrize("build", [
    lambda: C.rows(), lambda: C.global_scan(), lambda: C.scatter_gather(), lambda: C.scatter_gather(C.N3, C.N3),
    lambda: C.scatter_gather((1 << 20) + 3, 300 * 16384), lambda: C.scatter_gather(1 << 20, 1 << 16, F64),
    lambda: C.mc_greeks(4096, 64), lambda: C.matmul_grad(256), lambda: sx.program(1 << 20, 2.0),
])
@pytest.mark.parametrize("tune", ["", "scatter_windows=0", "scatter_local_max=0"])
def test_plan_launches_only_live_buffers(monkeypatch, build, tune):
    """Scratch shared between roots (a gather back reads the scatter's
    partition, window table included) stays allocated until its last use."""
    monkeypatch.setenv("CCHIP_TUNE", tune)
    _launch_uses_live_buffers(build())


def test_plan_liveness_over_random_scatter_shapes(monkeypatch):
    """Scatter/gather-back plans over random sizes, bin counts, dtypes and
    layout knobs (direct, tile-local, counted, two levels in windows or
    counted, fused slice step or not) launch only live buffers."""
    r = np.random.default_rng(11)
    for case in range(60):
        n = int(r.integers(1, 1 << 24))
        bins = int(2 ** r.uniform(0, 26.5)) + int(r.integers(0, 3))
        dt = [F32, F64, I32][case % 3]
        tune = ["", "scatter_windows=0", "scatter_fuse_back=0", "scatter_local_max=0", "scatter_two_level=0"][case % 5]
        monkeypatch.setenv("CCHIP_TUNE", tune)
        _launch_uses_live_buffers(C.scatter_gather(n, bins, dt))


def test_broadcast_read_in_place_by_its_consumers(monkeypatch):
    """A broadcast of a one-element tensor that the fusion plan
    materialises (it has two consumers) is read from its source by those
    consumers, and so is a map of broadcasts that does not use the element
    index; with no other reader and not an output, such a tensor's kernel
    is dropped and its buffer never allocated. An output broadcast, or one
    a matmul reads straight from memory, keeps its kernel;
    remat_broadcast=0 keeps every one."""
    s = D.scalar("s", F32)
    x = D.param("x", F32, (64, 64))
    b = D.broadcast((64, 64), s)
    g = Graph.create("bc", [("u", D.map2(D.add, b, x)), ("v", D.map2(D.mul, b, x))])
    bufs, ks, ops = parse(H.plan(g))
    assert [r for _, _, _, r in bufs].count("elided") == 1 and len(ks) == 2
    assert not any(o[0] in ("alloc", "free") and o[1] == [n for n, _, _, r in bufs if r == "elided"][0] for o in ops)
    _launch_uses_live_buffers(g)
    g2 = Graph.create("bc2", [("u", D.map2(D.add, b, x)), ("v", D.map2(D.mul, b, x)), ("b", b)])
    assert "elided" not in [r for _, _, _, r in parse(H.plan(g2))[0]] and len(kernels_of(g2)) == 3
    b2, x2 = D.broadcast((256, 256), s), D.param("x", F32, (256, 256))
    g3 = Graph.create("bc3", [("c", D.matmul(b2, x2)), ("v", D.map2(D.mul, b2, x2))])
    assert "matmul_mfma_f32_a0b0" in [t for _, t in kernels_of(g3)]
    assert "elided" not in [r for _, _, _, r in parse(H.plan(g3))[0]]
    _launch_uses_live_buffers(g3)
    # a map of broadcasts is one value too (elided); one that uses the
    # element index is not
    e = D.map(lambda v: D.exp(D.mul(v, D.const(F32, 0.5))), b)
    g4 = Graph.create("bc4", [("u", D.map2(D.add, e, x)), ("v", D.map2(D.mul, e, x))])
    assert [r for _, _, _, r in parse(H.plan(g4))[0]].count("elided") == 1 and len(kernels_of(g4)) == 2
    _launch_uses_live_buffers(g4)
    ei = D.map(lambda v: D.add(v, D.cast(F32, D.index())), b)
    g5 = Graph.create("bc5", [("u", D.map2(D.add, ei, x)), ("v", D.map2(D.mul, ei, x))])
    assert "elided" not in [r for _, _, _, r in parse(H.plan(g5))[0]] and len(kernels_of(g5)) == 3
    _launch_uses_live_buffers(g5)
    monkeypatch.setenv("CCHIP_TUNE", "remat_broadcast=0")
    assert "elided" not in [r for _, _, _, r in parse(H.plan(g))[0]] and len(kernels_of(g)) == 3


def _last_col_graph(rows, n, dtype, last=None, second=False):
    """A row scan whose rows' last elements (or the elements at column
    `last`) are gathered through a map, then summed."""
    x = D.param("x", dtype, (rows, n))
    p = D.scan_rows(D.add, D.const(dtype, 0), x)
    if second:
        y = D.param("y", dtype, (rows, n))
        p = D.map2(D.add, p, y)
    col = n - 1 if last is None else last
    idx = D.map(lambda i: D.add(D.mul(i, D.const(I32, n)), D.const(I32, col)), D.iota((rows,)))
    g = D.gather(idx, D.map(lambda v: D.mul(v, D.const(dtype, 3)), p))
    return Graph.create("lastcol", [("s", D.reduce(D.add, D.const(dtype, 0), g))])


def _reads(g):
    names, out = {}, {}
    for f in (l.split() for l in H.plan(g).splitlines()):
        if f[0] == "buffer":
            names[f[1]] = f[2]
        elif f[0] == "kernel":
            out[f[2]] = [names[a] for a in f[f.index("args") + 1:]]
    return out


def _mixed_row_last_graph(dtype):
    """Two row scans with side buffers, of rows 100 and 50 long; the first
    gather's source adds the second scan reshaped to the first's rows, so
    it reads that scan at p * 100 + 99, the last element of its row 2p + 1."""
    x = D.param("x", dtype, (2048, 100))
    y = D.param("y", dtype, (4096, 50))
    p = D.scan_rows(D.add, D.const(dtype, 5), x)
    q = D.scan_rows(D.add, D.const(dtype, 0), y)
    i2 = D.map(lambda i: D.add(D.mul(i, D.const(I32, 50)), D.const(I32, 49)), D.iota((4096,)))
    m = D.map2(D.add, p, D.reshape((2048, 100), q))
    i1 = D.map(lambda i: D.add(D.mul(i, D.const(I32, 100)), D.const(I32, 99)), D.iota((2048,)))
    return Graph.create("rowlast_mixed", [("last1", D.gather(i1, m)), ("last2", D.gather(i2, q))])


def test_row_last_side_buffer_only_for_rows_as_long():
    """A tensor with a side buffer, reached by another gather whose rows
    have another length, is read in its own buffer at the gathered index,
    not in its side buffer at the other gather's row index."""
    lines = [l.split() for l in H.plan(_mixed_row_last_graph(I32)).splitlines()]
    names = {f[1]: f[2] for f in lines if f[0] == "buffer"}
    kernels = [[names[a] for a in f[f.index("args") + 1:]] for f in lines if f[0] == "kernel"]
    scans = [k for k in kernels if k[0] in ("p_x", "p_y")]
    px_out, px_side = scans[0][1], scans[0][2]
    py_out, py_side = scans[1][1], scans[1][2]
    assert px_side.endswith("_last") and py_side.endswith("_last")
    readers = [k for k in kernels if k not in scans]
    last1 = [k for k in readers if px_side in k]
    assert len(last1) == 1 and last1[0][:2] == [px_side, py_out]
    assert [k[:1] for k in readers if k is not last1[0]] == [[py_side]]


def test_row_last_gather_reads_the_scans_side_buffer(monkeypatch):
    """A gather of every row's last element of a scan that folds one lane
    a row (config 5's final prices) reads a side buffer the scan writes,
    one value a row, instead of one cache line per row of the scan's
    output; other columns, tile-scanned rows and rowlast=0 keep the
    strided read."""
    from cudacaml_amd.examples import configs as C

    r = _reads(C.mc_paths(4096, 64))
    assert any(a.endswith("_last") for a in r["scan_rowseq"])
    assert any(a.endswith("_last") for a in r["reduce_split"])
    g = _last_col_graph(2048, 100, I32)
    r = _reads(g)
    side = [a for a in r["scan_rowseq"] if a.endswith("_last")]
    assert len(side) == 1 and side[0] in r["reduce_wave"]
    assert not any(a.endswith("_last") for a in _reads(_last_col_graph(2048, 100, I32, last=98))["scan_rowseq"])
    # a map over another tensor of the same shape between: that tensor is
    # read at the gathered index, the scan from its side buffer
    r = _reads(_last_col_graph(2048, 100, F32, second=True))
    assert "p_y" in r["reduce_wave"] and any(a.endswith("_last") for a in r["reduce_wave"])
    # rows long enough for the tile scan: no side buffer
    assert "_last" not in H.plan(_last_col_graph(2048, 4096, I32))
    # a materialised map root (the Greeks' paths tensor): its kernel writes
    # the side buffer, and the final-price map reads it
    lines = [l.split() for l in H.plan(C.mc_greeks(4096, 64)).splitlines()]
    side = [f[1] for f in lines if f[0] == "buffer" and f[2].endswith("_last")]
    users = [f[2] for f in lines if f[0] == "kernel" and side and side[0] in f[f.index("args") + 1:]]
    assert len(side) == 1 and users == ["map", "map"]
    monkeypatch.setenv("CCHIP_TUNE", "rowlast=0")
    assert "_last" not in H.plan(C.mc_paths(4096, 64))
    assert "_last" not in H.plan(C.mc_greeks(4096, 64))
