"""GPU parity: every kernel through the C ABI against the oracle, bit-exact.

int8 activations, act scale/sum and int32 dots must be identical to the CPU
restatement of src/i2s_gemm.c; f32 outputs must carry the same bits (the
epilogue is one IEEE division and one multiply, so the tolerance is zero,
tighter than the 1e-6 relative bound the path is allowed). Full-size
configurations are compared in full: the C oracle runs them in seconds.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def tensor(amd, seed, n_rows, n):
    return amd.synth_i2s(seed, n_rows, n)


def f32_bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def run_quant(amd, dev, x):
    x = np.ascontiguousarray(x, np.float32)
    m, n = x.shape
    bx = dev.put(x)
    bq = dev.alloc(m * n)
    ba = dev.alloc(8 * m)
    dev.quant_act(bx.vp, n, m, bq.vp, ba.vp)
    dev.sync()
    q = bq.download(np.int8, m * n).reshape(m, n)
    a = ba.download(np.uint8, 8 * m).view(np.dtype([("scale", "<f4"), ("sum", "<i4")]))
    for b in (bx, bq, ba):
        b.free()
    return q, a["scale"].astype(np.float32), a["sum"].astype(np.int32)


# ---------------------------------------------------------------------------
# quantiser
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,m", [(2560, 4), (6912, 3), (128, 1), (1000, 2), (1002, 2), (65536, 1)])
def test_quant_act_matches_oracle(amd, orc, dev, n, m):
    say("quant_act", n, m)
    rng = np.random.default_rng(n * 7 + m)
    x = (rng.standard_normal((m, n)) * rng.uniform(0.001, 100, (m, 1))).astype(np.float32)
    q, s, t = run_quant(amd, dev, x)
    q_o, s_o, t_o = orc.quant_act_rows(x)
    np.testing.assert_array_equal(q, q_o)
    assert f32_bits_equal(s, s_o)
    np.testing.assert_array_equal(t, t_o)


def test_quant_act_reproduces_the_upstream_lcg_kat(amd, orc, dev):
    for n, want_s, want_sum in ((2560, "42.3747139", 6643), (6912, "42.3359184", 1818)):
        say("quant_act lcg", n)
        q, s, t = run_quant(amd, dev, orc.lcg_activation(n)[None, :])
        assert s[0] == np.float32(float(want_s)) and t[0] == want_sum
        np.testing.assert_array_equal(q[0], orc.quant_act(orc.lcg_activation(n))[0])


def test_quant_act_edge_rows(amd, orc, dev):
    n = 256
    rows = [
        np.zeros(n, np.float32),                                            # scale 0
        np.where(np.arange(n) % 3 == 0, 2.0, -1.0).astype(np.float32),      # scale 63.5
        np.full(n, 1e-40, np.float32),                                      # denormal amax: 127/amax = inf
        np.where(np.arange(n) % 2 == 0, 3e38, -3e38).astype(np.float32),    # huge values
        np.linspace(-0.5, 0.5, n).astype(np.float32),                       # many ties after scaling
        np.where(np.arange(n) == 5, np.nan, 1.0).astype(np.float32),        # NaN is skipped by the max
    ]
    x = np.stack(rows)
    say("quant_act edges")
    q, s, t = run_quant(amd, dev, x)
    q_o, s_o, t_o = orc.quant_act_rows(x)
    np.testing.assert_array_equal(q, q_o)
    assert f32_bits_equal(s, s_o)
    np.testing.assert_array_equal(t, t_o)
    assert s[0] == 0 and s[1] == np.float32(63.5)


# ---------------------------------------------------------------------------
# GEMV (int32 dots) and the fused epilogue
# ---------------------------------------------------------------------------

SHAPES = [(2560, 2560), (6912, 2560), (2560, 6912), (640, 2560), (1, 128), (3, 384),
          (17, 1280), (1001, 6912), (77, 16384), (129, 65536)]

# (path, variant, lanes_per_row, waves, rows_per_wg[, slab_kib]): every kernel geometry.
# path 1 = streaming kernel (lanes per row, waves, rows per workgroup);
# path 2 = slab kernel (variant, KiB of weights per workgroup); 0 = automatic.
STREAMING = [(1, -1, 4, 1, 0), (1, -1, 8, 4, 0), (1, -1, 16, 2, 0), (1, -1, 8, 2, 48)]
SLABS = [(2, -1, 0, 0, 0), (2, 0, 0, 0, 0), (2, 1, 0, 0, 0), (2, -1, 0, 0, 0, 1), (2, -1, 0, 0, 0, 3),
         (2, 1, 0, 0, 0, 40), (2, -1, 0, 0, 0, 4096), (2, 1, 0, 0, 0, 2), (2, -1, 0, 0, 0, 5)]
GEOMETRIES = STREAMING + SLABS + [(0, -1, 0, 0, 0)]
# the slab kernel quantises f32 x in-kernel; these cover both of its variants
FUSED = [(2, -1, 0, 0, 0, 2), (2, 1, 0, 0, 0, 16), (2, -1, 0, 0, 0, 4096), (2, -1, 0, 0, 0, 3)]


@pytest.mark.parametrize("n_rows,n", SHAPES)
def test_gemv_int32_matches_oracle(amd, orc, dev, n_rows, n):
    say("gemv", n_rows, n)
    seed = amd.synth_seed(9, n_rows, n & 0xFFFF, 1)
    w = tensor(amd, seed, n_rows, n)
    rng = np.random.default_rng(n_rows + n)
    q = rng.integers(-128, 128, n, dtype=np.int8)
    want = orc.gemv(w, n_rows, n, q, orc.DOT_VNNI)
    bw, bq, bo = dev.put(w), dev.put(q), dev.alloc(4 * n_rows)
    try:
        for geom in GEOMETRIES:
            dev.set_tuning(*geom)
            bo.upload(np.full(n_rows, -7, np.int32))
            dev.gemv(bw.vp, n_rows, n, bq.vp, bo.vp)
            dev.sync()
            np.testing.assert_array_equal(bo.download(np.int32, n_rows), want, err_msg=f"geometry {geom}")
    finally:
        dev.set_tuning()
    for b in (bw, bq, bo):
        b.free()


def test_gemv_extreme_values_are_exact(amd, orc, dev):
    """All codes 2 against all -128 / +127 at the largest K."""
    n_rows, n = 64, 65536
    w = orc.pack_converter(np.full(n_rows * n, 2, np.uint8).reshape(n_rows, n)[0])
    w = np.concatenate([w[: n // 4]] * n_rows + [np.zeros(32, np.uint8)])
    bw = dev.put(w)
    for v in (-128, 127):
        say("gemv extremes", v)
        q = np.full(n, v, np.int8)
        bq, bo = dev.put(q), dev.alloc(4 * n_rows)
        dev.gemv(bw.vp, n_rows, n, bq.vp, bo.vp)
        dev.sync()
        assert (bo.download(np.int32, n_rows) == 2 * v * n).all()
        bq.free()
        bo.free()
    bw.free()


@pytest.mark.parametrize("n_rows,n", [(2560, 2560), (6912, 2560), (2560, 6912), (640, 2560), (5, 256)])
def test_linear_matches_oracle(amd, orc, dev, n_rows, n):
    """quantise -> GEMV -> epilogue, against orc_linear (src/forward.c:651-655)."""
    say("linear", n_rows, n)
    seed = amd.synth_seed(1, 0, n_rows & 0xFF, n & 0xFF)
    w = tensor(amd, seed, n_rows, n)
    x = amd.synth_normal(seed ^ 0xABC, n)
    y_o, q_o, d_o, s_o, t_o = orc.linear(w, n_rows, n, x, orc.DOT_VNNI)
    bw, bx = dev.put(w), dev.put(x)
    bq, ba, by, bi = dev.alloc(n), dev.alloc(8), dev.alloc(4 * n_rows), dev.alloc(4 * n_rows)
    try:
        for geom in [(0, -1, 0, 0, 0), (1, -1, 8, 2, 0), (1, -1, 16, 4, 0)] + FUSED:
            dev.set_tuning(*geom)
            for b, fill in ((bq, np.zeros(n, np.int8)), (ba, np.zeros(2, np.int32)),
                            (by, np.zeros(n_rows, np.float32)), (bi, np.zeros(n_rows, np.int32))):
                b.upload(fill)
            dev.linear(bw.vp, n_rows, n, bx.vp, bq.vp, ba.vp, by.vp)
            dev.gemv(bw.vp, n_rows, n, bq.vp, bi.vp)
            dev.sync()
            np.testing.assert_array_equal(bq.download(np.int8, n), q_o, err_msg=str(geom))
            a = ba.download(np.uint8, 8)
            assert a[:4].view(np.float32)[0] == s_o and a[4:].view(np.int32)[0] == t_o, geom
            np.testing.assert_array_equal(bi.download(np.int32, n_rows), d_o, err_msg=str(geom))
            assert f32_bits_equal(by.download(np.float32, n_rows), y_o), geom
        # without q / act outputs: library row scratch (streaming), or in-kernel
        for geom in [(0, -1, 0, 0, 0), (1, -1, 8, 2, 0)] + FUSED:
            dev.set_tuning(*geom)
            by.upload(np.zeros(n_rows, np.float32))
            dev.linear(bw.vp, n_rows, n, bx.vp, None, None, by.vp)
            dev.sync()
            assert f32_bits_equal(by.download(np.float32, n_rows), y_o), geom
    finally:
        dev.set_tuning()
    for b in (bw, bx, bq, ba, by, bi):
        b.free()


def test_zero_activation_gives_nan_like_the_reference(amd, orc, dev):
    n_rows, n = 64, 256
    w = tensor(amd, 77, n_rows, n)
    y_o = orc.linear(w, n_rows, n, np.zeros(n, np.float32))[0]
    assert np.isnan(y_o).all()
    bw, bx = dev.put(w), dev.put(np.zeros(n, np.float32))
    bq, ba, by = dev.alloc(n), dev.alloc(8), dev.alloc(4 * n_rows)
    say("linear zero row")
    dev.linear(bw.vp, n_rows, n, bx.vp, bq.vp, ba.vp, by.vp)
    dev.sync()
    assert np.isnan(by.download(np.float32, n_rows)).all()
    for b in (bw, bx, bq, ba, by):
        b.free()


# ---------------------------------------------------------------------------
# batched launches: the seven projections of a layer, one activation each
# ---------------------------------------------------------------------------

BLOCK = [("q", 2560, 2560, 0), ("k", 640, 2560, 0), ("v", 640, 2560, 0), ("o", 2560, 2560, 1),
         ("gate", 6912, 2560, 2), ("up", 6912, 2560, 2), ("down", 2560, 6912, 3)]


def test_batch_and_plan_over_a_block_match_oracle(amd, orc, dev):
    """QKV share one quantised activation, gate/up another (src/forward.c:645-773)."""
    say("batch block")
    xs = {0: 2560, 1: 2560, 2: 2560, 3: 6912}
    acts = {}
    bufs = []
    for a, n in xs.items():
        x = amd.synth_normal(1000 + a, n)
        q_o, s_o, t_o = orc.quant_act(x)
        bx, bq, ba = dev.put(x), dev.alloc(n), dev.alloc(8)
        dev.quant_act(bx.vp, n, 1, bq.vp, ba.vp)
        acts[a] = (bq, ba, q_o, s_o, t_o, bx)
        bufs += [bx, bq, ba]
    jobs, wants, outs = [], [], []
    for i, (name, n_rows, n, a) in enumerate(BLOCK):
        w = tensor(amd, amd.synth_seed(2, 0, 0, i), n_rows, n)
        bq, ba, q_o, s_o, t_o, _ = acts[a]
        d = orc.gemv(w, n_rows, n, q_o, orc.DOT_VNNI)
        wants.append((d, orc.epilogue_np(d, t_o, s_o, orc.scale(w, n_rows * n))))
        bw, by, bi = dev.put(w), dev.alloc(4 * n_rows), dev.alloc(4 * n_rows)
        outs.append((by, bi, n_rows))
        bufs += [bw, by, bi]
        # odd jobs quantise in-kernel from x, even jobs read the quantised row
        if i % 2:
            jobs.append(amd.GemvJob(bw.ptr, n_rows, n, acts[a][5].ptr, None, None, by.ptr, bi.ptr))
        else:
            jobs.append(amd.GemvJob(bw.ptr, n_rows, n, None, bq.ptr, ba.ptr, by.ptr, bi.ptr))
    # the numpy epilogue is checked against the C oracle here too
    d0 = wants[0][0]
    assert f32_bits_equal(wants[0][1][:64], orc.epilogue_rows(d0[:64], acts[0][4], acts[0][3],
                                                              orc.scale(tensor(amd, amd.synth_seed(2, 0, 0, 0), 2560, 2560), 2560 * 2560)))

    def check(tag):
        dev.sync()
        for (by, bi, n_rows), (d, y) in zip(outs, wants):
            np.testing.assert_array_equal(bi.download(np.int32, n_rows), d, err_msg=tag)
            assert f32_bits_equal(by.download(np.float32, n_rows), y), tag

    dev.gemv_batch(jobs)
    check("batch")
    plan = dev.plan(jobs)
    for rep in range(3):
        for by, bi, n_rows in outs:
            by.upload(np.zeros(n_rows, np.float32))
            bi.upload(np.zeros(n_rows, np.int32))
        say("plan replay", rep)
        dev.plan_run(plan)
        check(f"plan replay {rep}")
    dev.plan_destroy(plan)
    for b in bufs:
        b.free()


def test_mixed_plan_runs_every_launch_kind(amd, orc, dev):
    """One plan holding slab jobs (quantising in-kernel and pre-quantised) and
    K > 7168 jobs that take the streaming kernel, some after a quantiser
    launch."""
    specs = [(300, 2560, True), (64, 65536, True), (50, 16384, False), (129, 6912, True), (33, 20480, False)]
    jobs, checks, bufs = [], [], []
    for i, (n_rows, n, fused) in enumerate(specs):
        w = tensor(amd, amd.synth_seed(3, i, 0, 0), n_rows, n)
        x = amd.synth_normal(700 + i, n)
        y_o, q_o, d_o, s_o, t_o = orc.linear(w, n_rows, n, x, orc.DOT_VNNI)
        bw, bx, bq, ba = dev.put(w), dev.put(x), dev.alloc(n), dev.alloc(8)
        by, bi = dev.alloc(4 * n_rows), dev.alloc(4 * n_rows)
        bufs += [bw, bx, bq, ba, by, bi]
        if fused:
            jobs.append(amd.GemvJob(bw.ptr, n_rows, n, bx.ptr, bq.ptr, ba.ptr, by.ptr, bi.ptr))
        else:
            dev.quant_act(bx.vp, n, 1, bq.vp, ba.vp)
            jobs.append(amd.GemvJob(bw.ptr, n_rows, n, None, bq.ptr, ba.ptr, by.ptr, bi.ptr))
        checks.append((by, bi, bq, n_rows, n, y_o, d_o, q_o))
    try:
        for geom in [(0, -1, 0, 0, 0), (1, -1, 8, 2, 0)] + FUSED:
            say("mixed plan", geom)
            dev.set_tuning(*geom)
            plan = dev.plan(jobs)
            for rep in range(2):
                for by, bi, bq, n_rows, n, y_o, d_o, q_o in checks:
                    by.upload(np.zeros(n_rows, np.float32))
                    bi.upload(np.zeros(n_rows, np.int32))
                dev.plan_run(plan)
                dev.sync()
                for by, bi, bq, n_rows, n, y_o, d_o, q_o in checks:
                    np.testing.assert_array_equal(bi.download(np.int32, n_rows), d_o, err_msg=f"{n_rows}x{n} {geom}")
                    assert f32_bits_equal(by.download(np.float32, n_rows), y_o), (n_rows, n, geom)
                    np.testing.assert_array_equal(bq.download(np.int8, n), q_o)
            dev.plan_destroy(plan)
    finally:
        dev.set_tuning()
    say("mixed batch")
    dev.gemv_batch(jobs)
    dev.sync()
    for by, bi, bq, n_rows, n, y_o, d_o, q_o in checks:
        np.testing.assert_array_equal(bi.download(np.int32, n_rows), d_o)
    for b in bufs:
        b.free()


def test_checksum_and_copy_kernels(amd, dev):
    rng = np.random.default_rng(5)
    a = rng.integers(0, 2**32, 1 << 20, dtype=np.uint32)
    src, dst, part = dev.put(a), dev.alloc(a.nbytes), dev.alloc(4 * 64)
    say("copy / checksum")
    dev.copy(dst.vp, src.vp, a.nbytes)
    dev.checksum(src.vp, a.nbytes, part.vp, 64)
    dev.sync()
    np.testing.assert_array_equal(dst.download(np.uint32, a.size), a)
    assert int(np.bitwise_xor.reduce(part.download(np.uint32, 64))) == int(np.bitwise_xor.reduce(a))
    for b in (src, dst, part):
        b.free()


# ---------------------------------------------------------------------------
# the host-pointer kernel row and the dispatch table
# ---------------------------------------------------------------------------

def test_host_pointer_row_matches_oracle(amd, orc, dev):
    lib = amd.lib()
    n_rows, n = 1024, 2560
    w = tensor(amd, 4242, n_rows, n)
    amd.check(lib.sllm_gfx950_tensor_register(amd.ptr(w), n_rows, n), "register")
    try:
        x = amd.synth_normal(5, n)
        q = np.empty(n, np.int8)
        a = amd.Act()
        say("host row quant")
        lib.sllm_gfx950_i2s_quant_act(amd.ptr(x), n, amd.ptr(q), ctypes.byref(a))
        q_o, s_o, t_o = orc.quant_act(x)
        np.testing.assert_array_equal(q, q_o)
        assert np.float32(a.scale) == s_o and a.sum == t_o
        out = np.empty(n_rows, np.int32)
        say("host row gemv")
        lib.sllm_gfx950_i2s_gemv(amd.ptr(w), n_rows, n, amd.ptr(q), amd.ptr(out))
        want = orc.gemv(w, n_rows, n, q, orc.DOT_V3)
        np.testing.assert_array_equal(out, want)
        # an interior row range, as src/forward.c:190-194 hands to a worker
        part = np.empty(128, np.int32)
        wp = ctypes.c_void_p(w.ctypes.data + 64 * (n // 4))
        lib.sllm_gfx950_i2s_gemv(wp, 128, n, amd.ptr(q), amd.ptr(part))
        np.testing.assert_array_equal(part, want[64:192])
        d = lib.sllm_gfx950_i2s_dot(ctypes.c_void_p(w.ctypes.data + 7 * (n // 4)), amd.ptr(q), n)
        assert d == want[7]
        assert lib.sllm_gfx950_i2s_dot(None, amd.ptr(q), n) == 0
        # the row keeps a device copy of the vector quant_act returned: a
        # different buffer, and the same buffer rewritten by the host, are
        # read afresh
        q2 = np.random.default_rng(9).integers(-127, 128, n).astype(np.int8)
        want2 = orc.gemv(w, n_rows, n, q2, orc.DOT_V3)
        lib.sllm_gfx950_i2s_gemv(amd.ptr(w), n_rows, n, amd.ptr(q2), amd.ptr(out))
        np.testing.assert_array_equal(out, want2)
        lib.sllm_gfx950_i2s_quant_act(amd.ptr(x), n, amd.ptr(q), ctypes.byref(a))
        q[:] = q2
        lib.sllm_gfx950_i2s_gemv(amd.ptr(w), n_rows, n, amd.ptr(q), amd.ptr(out))
        np.testing.assert_array_equal(out, want2)
        lib.sllm_gfx950_i2s_quant_act(amd.ptr(x), n, amd.ptr(q), ctypes.byref(a))
        np.testing.assert_array_equal(q, q_o)
        # a shorter row (K 1024) through the same staging
        xs = amd.synth_normal(6, 1024)
        qs = np.empty(1024, np.int8)
        lib.sllm_gfx950_i2s_quant_act(amd.ptr(xs), 1024, amd.ptr(qs), ctypes.byref(a))
        qs_o, ss_o, ts_o = orc.quant_act(xs)
        np.testing.assert_array_equal(qs, qs_o)
        assert np.float32(a.scale) == ss_o and a.sum == ts_o
        lib.sllm_gfx950_i2s_quant_act(amd.ptr(x), n, amd.ptr(q), ctypes.byref(a))
        assert lib.sllm_gfx950_tensor_device(amd.ptr(w))
        assert not lib.sllm_gfx950_tensor_device(amd.ptr(q))
        # the dispatch table with the gfx950 row installed
        assert lib.sllm_kdispatch_select(b"gfx950") == 0
        assert lib.sllm_kdispatch_installed().contents.name == b"gfx950"
        out2 = np.zeros(n_rows, np.int32)
        lib.sllm_kdispatch_gemv(amd.ptr(w), n_rows, n, amd.ptr(q), amd.ptr(out2))
        np.testing.assert_array_equal(out2, want)
        lib.sllm_kdispatch_reset()
    finally:
        amd.check(lib.sllm_gfx950_tensor_unregister(amd.ptr(w)), "unregister")


def test_argument_errors_are_reported_not_launched(amd, dev):
    lib = amd.lib()
    b = dev.alloc(1 << 16)
    assert lib.sllm_gfx950_gemv(b.vp, 4, 200, b.vp, b.vp) == -34          # K % 128
    assert lib.sllm_gfx950_gemv(b.vp, 4, 65536 + 128, b.vp, b.vp) == -36  # K above the LDS limit
    assert lib.sllm_gfx950_gemv(b.at(4), 4, 128, b.vp, b.vp) == -1       # misaligned weights
    assert lib.sllm_gfx950_gemv_epilogue(b.vp, 4, 128, b.vp, None, b.vp) == -1
    assert lib.sllm_gfx950_set_tuning(0, -1, 5, 0, 0, 0) == -1         # lanes per row
    assert lib.sllm_gfx950_set_tuning(2, 2, 0, 0, 0, 0) == -1          # slab variants are 0 and 1
    assert lib.sllm_gfx950_set_tuning(2, -1, 0, 0, 0, -1) == -1        # slab KiB
    x = dev.alloc(4 * 128)
    job = amd.GemvJob(b.ptr, 4, 128, x.ptr, b.ptr, None, b.ptr, None)  # q without act
    assert lib.sllm_gfx950_gemv_batch(ctypes.byref(job), 1) == -1
    x.free()
    assert lib.sllm_gfx950_tensor_register(None, 4, 128) == -1
    b.free()


# ---------------------------------------------------------------------------
# full-size configurations, compared in full
# ---------------------------------------------------------------------------

def test_config1_rotated_sets_match_oracle(amd, orc, dev):
    """32 gate/up/down sets (425 MB of packed weights) in one plan, every dot
    and every output checked."""
    sets = 32
    shapes = [(6912, 2560), (6912, 2560), (2560, 6912)]
    pool = orc.Pool(16)
    jobs, checks, bufs = [], [], []
    for s in range(sets):
        x_up = amd.synth_normal(amd.synth_seed(1, s, 0, 100), 2560)
        x_dn = amd.synth_normal(amd.synth_seed(1, s, 0, 101), 6912)
        acts = []
        for x in (x_up, x_dn):
            n = x.size
            bx, bq, ba = dev.put(x), dev.alloc(n), dev.alloc(8)
            dev.quant_act(bx.vp, n, 1, bq.vp, ba.vp)
            acts.append((bq, ba) + orc.quant_act(x))
            bufs += [bx, bq, ba]
        for m, (n_rows, n) in enumerate(shapes):
            w = tensor(amd, amd.synth_seed(1, s, 0, m), n_rows, n)
            bq, ba, q_o, s_o, t_o = acts[0 if n == 2560 else 1]
            d = np.empty(n_rows, np.int32)
            pool.gemv(w, n_rows, n, q_o, d, orc.DOT_VNNI)
            checks.append((d, orc.epilogue_np(d, t_o, s_o, orc.scale(w, n_rows * n))))
            bw, by, bi = dev.put(w), dev.alloc(4 * n_rows), dev.alloc(4 * n_rows)
            bufs += [bw, by, bi]
            jobs.append(amd.GemvJob(bw.ptr, n_rows, n, None, bq.ptr, ba.ptr, by.ptr, bi.ptr))
    pool.close()
    say("config1 plan", len(jobs))
    plan = dev.plan(jobs)
    dev.plan_run(plan)
    dev.sync()
    for j, (d, y) in zip(jobs, checks):
        got_i = np.empty(j.n_rows, np.int32)
        amd.check(amd.lib().sllm_gfx950_d2h(amd.ptr(got_i), ctypes.c_void_p(j.rows_out), 4 * j.n_rows))
        got_y = np.empty(j.n_rows, np.float32)
        amd.check(amd.lib().sllm_gfx950_d2h(amd.ptr(got_y), ctypes.c_void_p(j.out), 4 * j.n_rows))
        np.testing.assert_array_equal(got_i, d)
        assert f32_bits_equal(got_y, y)
    dev.plan_destroy(plan)
    for b in bufs:
        b.free()


def test_thirty_block_plan_matches_oracle(amd, orc, dev):
    """Config 2 as the bench runs it: the decode GEMVs of 30 independently
    seeded BitNet-2B blocks (q/o 2560x2560, k/v 640x2560, gate/up 6912x2560,
    down 2560x6912; 521 MB), f32 N(0,1) inputs quantised in-kernel, as one
    plan -- a single launch of 210 GEMVs. Every raw int32 dot and every f32
    output of all 210 against the oracle (quantiser, VNNI dots over a pool of
    host threads, epilogue)."""
    say("thirty-block plan")
    pool = orc.Pool(16)
    jobs, checks, bufs = [], [], []
    try:
        for il in range(30):
            xs = {}
            for slot, n in ((0, 2560), (1, 2560), (2, 2560), (3, 6912)):
                x = amd.synth_normal(amd.synth_seed(2, 0, il, 200 + slot), n)
                bx = dev.put(x)
                bufs.append(bx)
                xs[slot] = (x, bx)
            for m, (name, n_rows, n, slot) in enumerate(BLOCK):
                w = tensor(amd, amd.synth_seed(2, 0, il, m), n_rows, n)
                bw, by, bi = dev.put(w), dev.alloc(4 * n_rows), dev.alloc(4 * n_rows)
                bufs += [bw, by, bi]
                jobs.append(amd.GemvJob(bw.ptr, n_rows, n, xs[slot][1].ptr, None, None, by.ptr, bi.ptr))
                checks.append((w, n_rows, n, xs[slot][0], by, bi, f"layer {il} {name}"))
        plan = dev.plan(jobs)
        dev.plan_run(plan)
        dev.sync()
        dev.plan_destroy(plan)
        say("thirty-block plan: checking 210 GEMVs")
        for w, n_rows, n, x, by, bi, what in checks:
            q, s, t = orc.quant_act(x)
            d = np.empty(n_rows, np.int32)
            pool.gemv(w, n_rows, n, q, d, orc.DOT_VNNI)
            np.testing.assert_array_equal(bi.download(np.int32, n_rows), d, err_msg=what)
            assert f32_bits_equal(by.download(np.float32, n_rows), orc.epilogue_np(d, t, s, orc.scale(w, n_rows * n))), what
    finally:
        pool.close()
        for b in bufs:
            b.free()
