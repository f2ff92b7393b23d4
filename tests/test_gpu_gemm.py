"""Several tokens against one tensor on int8 MFMA (sllm_gfx950_gemm /
sllm_gfx950_linear_batch) against the oracle, token by token.

The reference runs a chunk's projections one token at a time (each token
quantised on its own, its own GEMV and epilogue, src/forward.c:589-793), so
token t of the GEMM must equal the oracle's single-token linear of row t:
quantised row and scale / sum, every int32 dot and every f32 output, bit
for bit. Shapes: the BitNet-2B FFN pair (6912 x 2560, 2560 x 6912), a KV
projection (640 x 2560) and a ragged one (200 rows, K = 384); token counts
on and off the 16-token MFMA tile, up to the 512-token prefill chunk; every
tile shape the kernel has.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _case(amd, seed, n_rows, n, m):
    w = amd.synth_i2s(amd.synth_seed(3, seed, n_rows, n), n_rows, n)
    x = np.concatenate([amd.synth_normal(amd.synth_seed(3, seed, t, 1000 + n), n) for t in range(m)])
    return w, x.astype(np.float32)


def _run(amd, dev, w, n_rows, n, x, m):
    bw, bx = dev.put(w), dev.put(x)
    bq, ba = dev.alloc(m * n), dev.alloc(8 * m)
    by, bi = dev.alloc(4 * m * n_rows), dev.alloc(4 * m * n_rows)
    try:
        dev.linear_batch(bw.vp, n_rows, n, bx.vp, m, bq.vp, ba.vp, by.vp, bi.vp)
        dev.sync()
        y = by.download(np.float32, m * n_rows).reshape(m, n_rows)
        d = bi.download(np.int32, m * n_rows).reshape(m, n_rows)
        q = bq.download(np.int8, m * n).reshape(m, n)
        raw = ba.download(np.uint8, 8 * m).tobytes()
        act = np.frombuffer(raw, dtype=[("scale", "<f4"), ("sum", "<i4")])
        return y, d, q, act
    finally:
        for b in (bw, bx, bq, ba, by, bi):
            b.free()


def _check(orc, w, n_rows, n, x, m, y, d, q, act, label):
    for t in range(m):
        yo, qo, do, so, su = orc.linear(w, n_rows, n, x[t * n:(t + 1) * n])
        assert np.array_equal(q[t], qo), f"{label}: token {t} quantised row"
        assert act[t]["sum"] == su and bits(act[t]["scale"]) == bits(so), f"{label}: token {t} scale / sum"
        assert np.array_equal(d[t], do), f"{label}: token {t} dots"
        assert np.array_equal(bits(y[t]), bits(yo)), f"{label}: token {t} outputs"


SHAPES = [(6912, 2560), (2560, 6912), (640, 2560), (200, 384)]


@pytest.mark.parametrize("n_rows,n", SHAPES, ids=[f"{a}x{b}" for a, b in SHAPES])
@pytest.mark.parametrize("m", [1, 3, 4, 16, 17, 64, 100])
def test_gemm_matches_the_oracle_token_by_token(amd, orc, dev, n_rows, n, m):
    print(f"[gemm] {n_rows}x{n} m={m}", flush=True)
    w, x = _case(amd, 1, n_rows, n, m)
    y, d, q, act = _run(amd, dev, w, n_rows, n, x, m)
    _check(orc, w, n_rows, n, x, m, y, d, q, act, f"{n_rows}x{n} m={m}")


@pytest.mark.parametrize("tile", list(range(1, 16)))
def test_every_tile_shape_gives_the_same_bits(amd, orc, dev, tile):
    n_rows, n, m = 640, 2560, 37
    w, x = _case(amd, 2, n_rows, n, m)
    dev.set_gemm_tile(tile)
    try:
        y, d, q, act = _run(amd, dev, w, n_rows, n, x, m)
    finally:
        dev.set_gemm_tile(0)
    _check(orc, w, n_rows, n, x, m, y, d, q, act, f"tile {tile}")


@pytest.mark.parametrize("tile", list(range(1, 16)))
@pytest.mark.parametrize("n", [768, 6912])
def test_every_tile_shape_with_an_odd_count_of_super_steps(amd, orc, dev, tile, n):
    """K = 768 and 6912 are 3 and 27 super-steps of 256: the K-group tiles
    split them unevenly (two groups: the last iteration is group 0's alone;
    four groups: 27 = 6 x 4 + 3), and the partial sums still meet exactly."""
    n_rows, m = 320, 19
    w, x = _case(amd, 4, n_rows, n, m)
    dev.set_gemm_tile(tile)
    try:
        y, d, q, act = _run(amd, dev, w, n_rows, n, x, m)
    finally:
        dev.set_gemm_tile(0)
    _check(orc, w, n_rows, n, x, m, y, d, q, act, f"tile {tile} K {n}")


@pytest.mark.parametrize("tile", [0, 1, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15])
@pytest.mark.parametrize("m", [37, 512])
def test_several_tensors_in_one_launch(amd, orc, dev, tile, m):
    """Q, K and V (2560, 640, 640 rows) against the same quantised rows in
    one sllm_gfx950_gemm_multi launch: each job's outputs are the single
    GEMM's, and the oracle's token by token on the first and last token."""
    n = 2560
    rows = (2560, 640, 640)
    ws = [amd.synth_i2s(amd.synth_seed(3, 9, r, j), r, n) for j, r in enumerate(rows)]
    x = np.concatenate([amd.synth_normal(amd.synth_seed(3, 9, t, 2000), n) for t in range(m)]).astype(np.float32)
    bw = [dev.put(w) for w in ws]
    bx, bq, ba = dev.put(x), dev.alloc(m * n), dev.alloc(8 * m)
    outs = [(dev.alloc(4 * m * r), dev.alloc(4 * m * r)) for r in rows]
    ref = [(dev.alloc(4 * m * r), dev.alloc(4 * m * r)) for r in rows]
    dev.set_gemm_tile(tile)
    try:
        dev.quant_act(bx.vp, n, m, bq.vp, ba.vp)
        dev.gemm_multi([(bw[j].vp, rows[j], outs[j][0].vp, outs[j][1].vp) for j in range(3)], n, bq.vp, ba.vp, m)
        for j in range(3):
            dev.gemm(bw[j].vp, rows[j], n, bq.vp, ba.vp, m, ref[j][0].vp, ref[j][1].vp)
        dev.sync()
        for j, r in enumerate(rows):
            y = outs[j][0].download(np.float32, m * r).reshape(m, r)
            d = outs[j][1].download(np.int32, m * r).reshape(m, r)
            assert np.array_equal(bits(y), bits(ref[j][0].download(np.float32, m * r).reshape(m, r))), f"job {j}"
            assert np.array_equal(d, ref[j][1].download(np.int32, m * r).reshape(m, r)), f"job {j}"
            for t in (0, m - 1):
                yo, qo, do, so, su = orc.linear(ws[j], r, n, x[t * n:(t + 1) * n])
                assert np.array_equal(d[t], do) and np.array_equal(bits(y[t]), bits(yo)), f"job {j} token {t}"
    finally:
        dev.set_gemm_tile(0)
        for b in bw + [bx, bq, ba] + [b for p in outs + ref for b in p]:
            b.free()


@pytest.mark.parametrize("n_rows,n", [(6912, 2560), (2560, 6912)], ids=["gate_up", "down"])
def test_prefill_chunk_of_512_tokens(amd, orc, dev, n_rows, n):
    """The 512-token prefill shape: every token's quantised row, dots and
    outputs."""
    m = 512
    print(f"[gemm] prefill {n_rows}x{n}", flush=True)
    w, x = _case(amd, 3, n_rows, n, m)
    y, d, q, act = _run(amd, dev, w, n_rows, n, x, m)
    _check(orc, w, n_rows, n, x, m, y, d, q, act, f"prefill {n_rows}x{n}")


def test_zero_token_gives_nan_like_the_reference(amd, orc, dev):
    n_rows, n, m = 256, 256, 5
    w, x = _case(amd, 4, n_rows, n, m)
    x[2 * n:3 * n] = 0.0
    y, d, q, act = _run(amd, dev, w, n_rows, n, x, m)
    assert np.isnan(y[2]).all() and (d[2] == 0).all() and act[2]["scale"] == 0
    _check(orc, w, n_rows, n, x, 2, y, d, q, act, "rows before the zero token")


def test_gemm_refuses_bad_arguments(amd, dev):
    lib = amd.lib()
    w = dev.put(amd.synth_i2s(1, 64, 256))
    q, a, o = dev.alloc(256 * 2), dev.alloc(16), dev.alloc(4 * 64 * 2)
    try:
        assert lib.sllm_gfx950_gemm(w.vp, 64, 200, q.vp, a.vp, 2, o.vp, None) == -34    # K % 128
        assert lib.sllm_gfx950_gemm(w.vp, 64, 256, q.vp, None, 2, o.vp, None) == -1     # epilogue without act
        assert lib.sllm_gfx950_gemm(w.vp, 64, 256, q.vp, a.vp, 2, None, None) == -1     # no output
        assert lib.sllm_gfx950_gemm(w.vp, 64, 256, q.vp, a.vp, 0, o.vp, None) == 0      # nothing to do
        assert lib.sllm_gfx950_set_gemm_tile(16) == -1
    finally:
        for b in (w, q, a, o):
            b.free()


@pytest.mark.parametrize("tile", [0, 6, 7, 10, 11, 13])
@pytest.mark.parametrize("m", [1, 3, 4, 16, 17, 64, 100])
def test_gemm_plan_over_many_tensors(amd, orc, dev, tile, m):
    """A GEMM plan of seven tensors with their own K (2560 and 6912), token
    rows and outputs, one launch: each job's dots and outputs are the single
    sllm_gfx950_gemm's for it, and the oracle's on the first and last token;
    the automatic tile (0: the stream up to four tokens) and every plan tile
    forced, from one token up. Rows 90 (not a multiple of four) take the
    element-wise stores."""
    shapes = [(640, 2560), (2560, 6912), (384, 2560), (128, 6912), (2560, 2560), (64, 2560), (90, 2560)]
    ws = [amd.synth_i2s(amd.synth_seed(8, j, r, k), r, k) for j, (r, k) in enumerate(shapes)]
    xs = [np.concatenate([amd.synth_normal(amd.synth_seed(8, j, t, 3000), k) for t in range(m)]).astype(np.float32)
          for j, (r, k) in enumerate(shapes)]
    bw = [dev.put(w) for w in ws]
    bx = [dev.put(x) for x in xs]
    bq = [dev.alloc(m * k) for r, k in shapes]
    ba = [dev.alloc(8 * m) for _ in shapes]
    outs = [(dev.alloc(4 * m * r), dev.alloc(4 * m * r)) for r, k in shapes]
    refs = [(dev.alloc(4 * m * r), dev.alloc(4 * m * r)) for r, k in shapes]
    print(f"[gemm plan] tile {tile} m={m}", flush=True)
    dev.set_gemm_tile(tile)
    plan = None
    try:
        for j, (r, k) in enumerate(shapes):
            dev.quant_act(bx[j].vp, k, m, bq[j].vp, ba[j].vp)
        # job 1 writes only raw dots, job 4 only the epilogue
        plan = dev.gemm_plan([(bw[j].vp, r, k, bq[j].vp, ba[j].vp, None if j == 1 else outs[j][0].vp,
                               None if j == 4 else outs[j][1].vp) for j, (r, k) in enumerate(shapes)], m)
        dev.gemm_plan_run(plan)
        dev.set_gemm_tile(0)
        for j, (r, k) in enumerate(shapes):
            dev.gemm(bw[j].vp, r, k, bq[j].vp, ba[j].vp, m, refs[j][0].vp, refs[j][1].vp)
        dev.sync()
        for j, (r, k) in enumerate(shapes):
            yr = refs[j][0].download(np.float32, m * r).reshape(m, r)
            dr = refs[j][1].download(np.int32, m * r).reshape(m, r)
            if j != 1:
                y = outs[j][0].download(np.float32, m * r).reshape(m, r)
                assert np.array_equal(bits(y), bits(yr)), f"job {j}"
            if j != 4:
                d = outs[j][1].download(np.int32, m * r).reshape(m, r)
                assert np.array_equal(d, dr), f"job {j}"
            for t in (0, m - 1):
                yo, qo, do, so, su = orc.linear(ws[j], r, k, xs[j][t * k:(t + 1) * k])
                assert np.array_equal(dr[t], do) and np.array_equal(bits(yr[t]), bits(yo)), f"job {j} token {t}"
    finally:
        dev.set_gemm_tile(0)
        if plan is not None:
            dev.gemm_plan_destroy(plan)
        for b in bw + bx + bq + ba + [b for p in outs + refs for b in p]:
            b.free()


@pytest.mark.parametrize("m", [1, 3, 4])
def test_streamed_plan_runs_of_many_tiles(amd, orc, dev, m):
    """Up to four tokens a plan streams: its 128-row tiles are cut into runs,
    one per workgroup, and each run keeps one ring of copies going across
    its tiles' boundaries, storing a tile's outputs during the next tile's
    first iteration (i2s_kernels.hip: gemm_stream_body). 100 jobs over five
    shapes -- K = 256, 768, 2560, 6912; rows 130 and 90 not multiples of
    128, 90 not of 4 -- make 620 tiles on 256 runs, so runs go from one K to
    another and end on partial tiles. Every job's dots and outputs are the
    single sllm_gfx950_gemm's for its tensor and tokens, and those the
    oracle's on the first and last token."""
    shapes = [(640, 2560), (384, 768), (130, 256), (2560, 6912), (90, 2560)]
    ws = [amd.synth_i2s(amd.synth_seed(11, j, r, k), r, k) for j, (r, k) in enumerate(shapes)]
    xs = [np.concatenate([amd.synth_normal(amd.synth_seed(11, j, t, 5000), k) for t in range(m)]).astype(np.float32)
          for j, (r, k) in enumerate(shapes)]
    bw = [dev.put(w) for w in ws]
    bx = [dev.put(x) for x in xs]
    bq = [dev.alloc(m * k) for r, k in shapes]
    ba = [dev.alloc(8 * m) for _ in shapes]
    refs = [(dev.alloc(4 * m * r), dev.alloc(4 * m * r)) for r, k in shapes]
    n_jobs = 100
    outs = [(dev.alloc(4 * m * shapes[i % 5][0]), dev.alloc(4 * m * shapes[i % 5][0])) for i in range(n_jobs)]
    print(f"[streamed plan] m={m}", flush=True)
    plan = None
    try:
        for j, (r, k) in enumerate(shapes):
            dev.quant_act(bx[j].vp, k, m, bq[j].vp, ba[j].vp)
            dev.gemm(bw[j].vp, r, k, bq[j].vp, ba[j].vp, m, refs[j][0].vp, refs[j][1].vp)
        # a third of the jobs write only raw dots, a third only the epilogue
        jobs = []
        for i in range(n_jobs):
            j = i % 5
            r, k = shapes[j]
            jobs.append((bw[j].vp, r, k, bq[j].vp, ba[j].vp, None if i % 3 == 0 else outs[i][0].vp,
                         None if i % 3 == 1 else outs[i][1].vp))
        plan = dev.gemm_plan(jobs, m)
        dev.gemm_plan_run(plan)
        dev.sync()
        for j, (r, k) in enumerate(shapes):
            yr = refs[j][0].download(np.float32, m * r).reshape(m, r)
            dr = refs[j][1].download(np.int32, m * r).reshape(m, r)
            for t in (0, m - 1):
                yo, qo, do, so, su = orc.linear(ws[j], r, k, xs[j][t * k:(t + 1) * k])
                assert np.array_equal(dr[t], do) and np.array_equal(bits(yr[t]), bits(yo)), f"shape {j} token {t}"
        for i in range(n_jobs):
            r, k = shapes[i % 5]
            yr = refs[i % 5][0].download(np.float32, m * r).reshape(m, r)
            dr = refs[i % 5][1].download(np.int32, m * r).reshape(m, r)
            if i % 3 != 0:
                y = outs[i][0].download(np.float32, m * r).reshape(m, r)
                assert np.array_equal(bits(y), bits(yr)), f"job {i}"
            if i % 3 != 1:
                d = outs[i][1].download(np.int32, m * r).reshape(m, r)
                assert np.array_equal(d, dr), f"job {i}"
    finally:
        if plan is not None:
            dev.gemm_plan_destroy(plan)
        for b in bw + bx + bq + ba + [b for p in refs + outs for b in p]:
            b.free()


def test_gemm_plan_refuses_bad_jobs(amd, dev):
    lib = amd.lib()
    w = dev.put(amd.synth_i2s(1, 64, 384))
    q, a, o = dev.alloc(384 * 2), dev.alloc(16), dev.alloc(4 * 64 * 2)
    p = ctypes.c_void_p()
    try:
        def create(job, m=2):
            arr = (amd.GemmPlanJob * 1)(amd.GemmPlanJob(*job))
            return lib.sllm_gfx950_gemm_plan_create(arr, 1, m, ctypes.byref(p))
        assert create((w.vp, 64, 384, q.vp, a.vp, o.vp, None)) == -34        # K % 256
        assert create((w.vp, 64, 256, q.vp, None, o.vp, None)) == -1         # epilogue without act
        assert create((w.vp, 64, 256, q.vp, a.vp, None, None)) == -1         # no output
        assert create((w.vp, 64, 256, None, a.vp, o.vp, None)) == -1         # no q
        assert create((w.vp, 64, 256, q.vp, a.vp, o.vp, None), m=0) == -36
        assert lib.sllm_gfx950_gemm_plan_run(None) == -1
    finally:
        for b in (w, q, a, o):
            b.free()

