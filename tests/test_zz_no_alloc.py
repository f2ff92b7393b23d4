"""sllm_gfx950_gemv_batch_noalloc: the GEMV batch whose tables and
quantised rows live in a static device array. Through the C ABI, its outputs
equal sllm_gfx950_gemv_batch's (the existing entry point, itself pinned to
the oracle by the parity tests) bit for bit, on two calls in a row -- the
second with a smaller batch, so stale tables or rows from the first would
show -- and it refuses a batch the array cannot hold before enqueueing
anything."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _batch(amd, dev, specs, seed):
    """Device buffers for `specs` [(n_rows, K, kind)]: kind "x" quantises an
    f32 activation in the launch (no q / act given), "xq" also writes q / act,
    "q" takes a quantised row. Returns (jobs for the no-allocation call, jobs
    for the reference call, output readers, buffers)."""
    bufs, jobs_a, jobs_b, outs = [], [], [], []
    for i, (n_rows, k, kind) in enumerate(specs):
        w = amd.synth_i2s(amd.synth_seed(7, seed, i, 0), n_rows, k)
        x = amd.synth_normal(amd.synth_seed(7, seed, i, 1), k)
        bw, bx = dev.put(w), dev.put(x)
        bufs += [bw, bx]
        pair = []
        for _ in range(2):
            by, bi = dev.alloc(4 * n_rows), dev.alloc(4 * n_rows)
            bq, ba = dev.alloc(k), dev.alloc(8)
            bufs += [by, bi, bq, ba]
            pair.append((by, bi, bq, ba))
        if kind == "q":                              # a quantised row, made once, shared by both calls
            dev.quant_act(bx.vp, k, 1, pair[0][2].vp, pair[0][3].vp)
            dev.sync()
            q = pair[0][2].download(np.int8, k)
            a = pair[0][3].download(np.uint8, 8)
            pair[1][2].upload(q)
            pair[1][3].upload(a)
        for (by, bi, bq, ba), jobs in zip(pair, (jobs_a, jobs_b)):
            if kind == "x":
                jobs.append(amd.GemvJob(bw.ptr, n_rows, k, bx.ptr, None, None, by.ptr, bi.ptr))
            elif kind == "xq":
                jobs.append(amd.GemvJob(bw.ptr, n_rows, k, bx.ptr, bq.ptr, ba.ptr, by.ptr, bi.ptr))
            else:
                jobs.append(amd.GemvJob(bw.ptr, n_rows, k, None, bq.ptr, ba.ptr, by.ptr, bi.ptr))
        outs.append((n_rows, k, kind, pair))
    return jobs_a, jobs_b, outs, bufs


def _compare(outs, label):
    for i, (n_rows, k, kind, pair) in enumerate(outs):
        (ya, ia, qa, aa), (yb, ib, qb, ab) = pair
        got_y, want_y = ya.download(np.float32, n_rows), yb.download(np.float32, n_rows)
        assert np.array_equal(ia.download(np.int32, n_rows), ib.download(np.int32, n_rows)), f"{label} job {i}: dots"
        assert np.array_equal(got_y.view(np.uint32), want_y.view(np.uint32)), f"{label} job {i}: outputs"
        if kind == "xq":
            assert np.array_equal(qa.download(np.int8, k), qb.download(np.int8, k)), f"{label} job {i}: q"
            assert np.array_equal(aa.download(np.uint8, 8), ab.download(np.uint8, 8)), f"{label} job {i}: act"


def test_noalloc_batch_equals_the_allocating_batch(amd, dev):
    # slab jobs (K <= 7168) quantising in-kernel, writing q / act, reading a
    # quantised row; streaming jobs (K > 7168) whose quantised rows go into
    # the array, or into their own q / act
    first = [(2560, 2560, "x"), (640, 2560, "x"), (6912, 2560, "xq"), (2560, 6912, "q"),
             (300, 8192, "x"), (129, 16384, "x"), (64, 8192, "xq"), (1000, 1024, "q")]
    second = [(100, 8192, "x"), (640, 2560, "x")]
    for label, specs, seed in (("first call", first, 1), ("second, smaller call", second, 2)):
        print(f"[no-alloc] {label}: {len(specs)} jobs", flush=True)
        jobs_a, jobs_b, outs, bufs = _batch(amd, dev, specs, seed)
        try:
            dev.gemv_batch_noalloc(jobs_a)
            dev.gemv_batch(jobs_b)
            dev.sync()
            _compare(outs, label)
        finally:
            for b in bufs:
                b.free()


def test_noalloc_batch_refuses_what_the_array_cannot_hold(amd, dev):
    lib = amd.lib()
    n_max = 1024                                   # SLLM_GFX950_NOALLOC_MAX_JOBS
    k = 65536
    w = amd.synth_i2s(amd.synth_seed(7, 9, 0, 0), 16, k)
    bw, by = dev.put(w), dev.alloc(4 * 16)
    bx = dev.alloc(4 * k * 16)
    try:
        job = amd.GemvJob(bw.ptr, 16, k, bx.ptr, None, None, by.ptr, None)
        many = (amd.GemvJob * (n_max + 1))(*([job] * (n_max + 1)))
        assert lib.sllm_gfx950_gemv_batch_noalloc(many, n_max + 1) == -36
        # sixteen distinct 65536-wide activations need 16 x 65792 bytes of
        # quantised rows, more than the 1 MiB array
        rows = (amd.GemvJob * 16)(*[amd.GemvJob(bw.ptr, 16, k, bx.ptr + 4 * k * i, None, None, by.ptr, None)
                                    for i in range(16)])
        assert lib.sllm_gfx950_gemv_batch_noalloc(rows, 16) == -36
        assert b"the array holds" in lib.sllm_gfx950_last_error()
        assert lib.sllm_gfx950_gemv_batch_noalloc(None, 0) == 0
    finally:
        for b in (bw, by, bx):
            b.free()
